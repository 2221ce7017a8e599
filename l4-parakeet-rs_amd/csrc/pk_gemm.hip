// Instantiations and the launcher of the byte-tile GEMM engine.
#include <cstdlib>
#include <mutex>

#include "pk_gemm3.hpp"
#include "pk_kernels.hpp"

namespace pk {

int cu_count() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return cus;
}

template <int F, int E>
static int launch_one(const GemmArgs& a, hipStream_t s) {
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void*)gemm_kernel<F, E>, hipFuncAttributeMaxDynamicSharedMemorySize, Layout<F>::kBytes);
    });
    if (attr != hipSuccess) {
        set_error("hipFuncSetAttribute(LDS %d bytes) failed: %s", Layout<F>::kBytes, hipGetErrorString(attr));
        return -3;
    }
    const int tiles = ((a.m + kBlockM - 1) / kBlockM) * ((a.n + kBlockN - 1) / kBlockN);
    const int cus = cu_count();
    // one persistent workgroup per CU; a multiple of 8 keeps the XCD mapping
    const int grid = tiles < cus ? tiles : cus - cus % 8;
    hipLaunchKernelGGL((gemm_kernel<F, E>), dim3(grid), dim3(kThreads), Layout<F>::kBytes, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("gemm launch (fmt %d, epi %d) failed: %s", F, E, hipGetErrorString(e));
        return -3;
    }
    return 0;
}

// The occupancy-2 engine: two workgroups per CU, 32*kAI x 128 tiles.
template <int F, int E, int kAI>
static int launch_two(const GemmArgs& a, hipStream_t s) {
    using L = g3::L3<F, kAI>;
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void*)g3::gemm3_kernel<F, E, kAI>, hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes);
    });
    if (attr != hipSuccess) {
        set_error("hipFuncSetAttribute(LDS %d bytes) failed: %s", L::kBytes, hipGetErrorString(attr));
        return -3;
    }
    const int tiles = ((a.m + L::kBM - 1) / L::kBM) * ((a.n + g3::kBN - 1) / g3::kBN);
    const int slots = 2 * cu_count();
    // two persistent workgroups per CU; a multiple of 8 keeps the XCD mapping
    const int grid = tiles < slots ? tiles : slots - slots % 8;
    hipLaunchKernelGGL((g3::gemm3_kernel<F, E, kAI>), dim3(grid), dim3(g3::kThreads), L::kBytes, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("gemm launch (fmt %d, epi %d) failed: %s", F, E, hipGetErrorString(e));
        return -3;
    }
    return 0;
}

static int forced_tile_rows();

// One tile per workgroup with an S-stage ring (grids of at most one tile per CU).
template <int F, int E, int kAI, int kOcc = 1>
static int launch_ring(const GemmArgs& a, hipStream_t s) {
    using L = g3::LS<F, kAI, kOcc>;
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void*)g3::gemm3_ring_kernel<F, E, kAI, kOcc>, hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes);
    });
    if (attr != hipSuccess) {
        set_error("hipFuncSetAttribute(LDS %d bytes) failed: %s", L::kBytes, hipGetErrorString(attr));
        return -3;
    }
    const int tiles = ((a.m + L::kBM - 1) / L::kBM) * ((a.n + g3::kBN - 1) / g3::kBN);
    hipLaunchKernelGGL((g3::gemm3_ring_kernel<F, E, kAI, kOcc>), dim3(tiles), dim3(g3::kThreads), L::kBytes, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("gemm launch (fmt %d, epi %d) failed: %s", F, E, hipGetErrorString(e));
        return -3;
    }
    return 0;
}

// The ring kernel with two waves per SIMD (FP8 / INT8, 64- or 128-row tiles;
// measured slower for INT4-g128 x fp16 on 96-row tiles, split 2 : 1, 19.6 ->
// 22.6 us, and for INT4-g128 x INT8 on 128-row tiles against its two 64-row
// ring workgroups per CU, 13.4 -> 13.9 us).
template <int F, int E, int kAI>
static int launch_ring8(const GemmArgs& a, hipStream_t s) {
    using L = g3::LS<F, kAI, 1>;
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void*)g3::gemm3_ring8_kernel<F, E, kAI>, hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes);
    });
    if (attr != hipSuccess) {
        set_error("hipFuncSetAttribute(LDS %d bytes) failed: %s", L::kBytes, hipGetErrorString(attr));
        return -3;
    }
    const int tiles = ((a.m + L::kBM - 1) / L::kBM) * ((a.n + g3::kBN - 1) / g3::kBN);
    hipLaunchKernelGGL((g3::gemm3_ring8_kernel<F, E, kAI>), dim3(tiles), dim3(2 * g3::kThreads), L::kBytes, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("gemm launch (fmt %d, epi %d) failed: %s", F, E, hipGetErrorString(e));
        return -3;
    }
    return 0;
}

// One 32-row tile per workgroup with K split in four parts, each part's
// ring shared by kCH waves that take 128 / kCH columns each (INT4-g128
// formats, grids that take 32-row ring tiles, K >= 1024).  kCH = 4 (16 waves)
// by measurement: C3 FF2 at T = 750 x INT8 / x fp16 14.8 / 23.4 us with 8
// waves, 13.5 / 22.8 with 16 (4 waves, one per SIMD: 17.0 / 24.9).
template <int F, int E, int kCH>
static int launch_splitk(const GemmArgs& a, hipStream_t s) {
    using L = g3::LK<F, kCH>;
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void*)g3::gemm3_splitk_kernel<F, E, kCH>, hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes);
    });
    if (attr != hipSuccess) {
        set_error("hipFuncSetAttribute(LDS %d bytes) failed: %s", L::kBytes, hipGetErrorString(attr));
        return -3;
    }
    const int tiles = ((a.m + L::kBM - 1) / L::kBM) * ((a.n + g3::kBN - 1) / g3::kBN);
    hipLaunchKernelGGL((g3::gemm3_splitk_kernel<F, E, kCH>), dim3(tiles), dim3(L::kThreads), L::kBytes, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("gemm launch (fmt %d, epi %d) failed: %s", F, E, hipGetErrorString(e));
        return -3;
    }
    return 0;
}

// Formats with a ring variant and the tile rows it takes for an m x n
// output: the smallest tile (32, 64, 96 (INT4-g128 x fp16 only) or 128 rows)
// whose tile count fits one workgroup per CU, or 0 when even 128-row tiles
// outnumber the CUs.
static bool has_ring(int fmt, int epi) {
    return (fmt == FMT_FP8 || fmt == FMT_I8 || fmt == FMT_G128A8 || fmt == FMT_G128A16) && epi != EPI_GLU && epi != EPI_F8_24 &&
           epi != EPI_I8S;
}
template <int F> static int ring_stages_of(int kAI) {
    return kAI == 1 ? g3::LS<F, 1>::kS : (kAI == 2 ? g3::LS<F, 2>::kS : (kAI == 3 ? g3::LS<F, 3>::kS : g3::LS<F, 4>::kS));
}
static int ring_stages(int fmt, int kAI) {
    switch (fmt) {
    case FMT_FP8: return ring_stages_of<FMT_FP8>(kAI);
    case FMT_I8: return ring_stages_of<FMT_I8>(kAI);
    case FMT_G128A8: return ring_stages_of<FMT_G128A8>(kAI);
    default: return ring_stages_of<FMT_G128A16>(kAI);
    }
}
// INT4-g128 x INT8 grids whose ring tiles would be 128 rows but whose 64-row
// tiles fit two workgroups per CU run 64-row ring tiles two per CU (3-stage
// rings of 16 KiB stages, 68 KiB each): twice the workgroups for the chain of
// K-steps (C3 FF1 at T = 750, 384 tiles: 16.6 -> 14.2 us).  Measured and not
// taken for INT8 (C1: 13.4 vs 13.5 us) and INT4-g128 x fp16 (23.2 -> 24.9 us).
static int ring_rows(int fmt, int m, int n);
static bool ring_occ2(int fmt, int m, int n) {
    if (fmt != FMT_G128A8 || ring_rows(fmt, m, n) != 128) return false;
    return ((m + 63) / 64) * ((n + g3::kBN - 1) / g3::kBN) <= 2 * cu_count();
}

// The K split of a launch: 4 (gemm3_splitk_kernel) for the INT4-g128 formats
// when the ring takes 32-row tiles and K >= 1024 (C3 FF2 at T = 750: the ring
// kernel's 64 / 32 K-steps per tile become 16 / 8 per part), else 1.
static int k_split(int fmt, int epi, int m, int n, int k) {
    if ((fmt != FMT_G128A8 && fmt != FMT_G128A16) || !has_ring(fmt, epi) || k < 1024) return 1;
    return ring_rows(fmt, m, n) == 32 ? 4 : 1;
}
static int ring_rows(int fmt, int m, int n) {
    if (forced_tile_rows() != 0) return 0;
    const int cols = (n + g3::kBN - 1) / g3::kBN;
    for (int rows = 32; rows <= 128; rows += 32) {
        // 96-row tiles (every CU busy where 128-row tiles leave a quarter
        // idle, e.g. 750 x 4096: 256 vs 192 tiles) pay for INT4-g128 x fp16
        // only (C3 FF1 at T = 750: 22.7 -> 19.2 us); measured slower for INT8
        // (12.8 -> 14.3 us) and INT4-g128 x INT8, equal for FP8
        if (rows == 96 && fmt != FMT_G128A16) continue;
        if (((m + rows - 1) / rows) * cols <= cu_count()) return rows;
    }
    return 0;
}

// Tile rows of the occupancy-2 engine for an m x n output: 64-row tiles when
// 128-row tiles would number at most a quarter of the CUs (INT4-g128 x INT8
// FF2 at T = 750: 59 -> 48 us); 128-row tiles (twice as many) when 256-row
// tiles would fill at most half of the two-per-CU workgroup slots, by
// measurement: C1, attention-out / FF2 and the sparse FF2 at T = 7500 and the
// INT4-g128 x INT8 linears at T = 750 run 18-29 % faster; grids of 256-row
// tiles filling more than half the slots run slower with 128 rows (pw1 at
// T = 7500: 480 tiles, -5 %).  PK_GEMM_TILE_ROWS = 64, 128 or 256 forces one
// size (measurement only); any other value is rejected at the first launch.
static int forced_tile_rows() {
    static const int force = [] {
        const char* v = getenv("PK_GEMM_TILE_ROWS");
        if (!v || !*v) return 0;
        const int r = atoi(v);
        return (r == 64 || r == 128 || r == 256) ? r : -1;
    }();
    return force;
}

// Tile rows of the occupancy-2 engine.  Grids whose 256-row tiles would not
// give every CU one take 128 (or, for a quarter of the CUs, 64) rows.  When
// both heights fill the chip, the one with fewer whole rounds of the 2 x CUs
// persistent workgroups wins by a margin, a 128-row tile costing half a
// 256-row one times its measured overhead (the smaller tile moves more operand bytes per MFMA:
// 9 % for FP8 / INT8, 22 % for INT4-g128 x INT8 at T = 45000).  E.g. QKV at
// T = 7500: 720 tiles of 256 rows take 2 rounds of 512 (the second 40 % full),
// 1416 of 128 rows 3 rounds of half the cost.
static int byte_tile_rows(int fmt, int m, int n) {
    const int tiles256 = ((m + 255) / 256) * ((n + g3::kBN - 1) / g3::kBN);
    const int tiles128 = ((m + 127) / 128) * ((n + g3::kBN - 1) / g3::kBN);
    const int force = forced_tile_rows();
    if (force > 0) return force;
    const int cus = cu_count(), slots = 2 * cus;
    if (4 * tiles128 <= cus) return 64;
    if (tiles256 <= cus) return 128;
    const int r256 = (tiles256 + slots - 1) / slots, r128 = (tiles128 + slots - 1) / slots;
    const float overhead = fmt == FMT_G128A8 ? 1.22f : 1.09f;
    return 0.5f * overhead * (float)r128 < 0.95f * (float)r256 ? 128 : 256;  // a clear win only
}

// Engine per format, by measurement on MI355X: the occupancy-2 engine for the
// byte formats, the 256x256 engine for fp16 activations (FP16, G128A16, Q4K),
// whose 64-K steps make its per-step barriers relatively more costly.
// Grids too small to give each CU a 256 x 256 tile take the occupancy-2
// engine's 128 x 128 tiles for the fp16-activation formats too.  Returns the
// tile rows and sets *cols (256 for the one-workgroup engine, 128 otherwise).
static int tile_plan(int fmt, int epi, int m, int n, int* cols, int* stages) {
    *cols = g3::kBN;
    *stages = 2;
    if (has_ring(fmt, epi)) {
        if (ring_occ2(fmt, m, n)) {
            *stages = g3::LS<FMT_G128A8, 2, 2>::kS;
            return 64;
        }
        const int r = ring_rows(fmt, m, n);
        if (r) {
            *stages = ring_stages(fmt, r / 32);
            return r;
        }
    }
    if (fmt == FMT_Q4K || (fmt == FMT_FP8 && epi == EPI_GLU)) {
        *cols = kBlockN;
        return kBlockM;
    }
    if (fmt == FMT_F16 || fmt == FMT_G128A16) {
        const int tiles256 = ((m + 255) / 256) * ((n + g3::kBN - 1) / g3::kBN);
        const int tiles128 = ((m + 127) / 128) * ((n + g3::kBN - 1) / g3::kBN);
        if (4 * tiles128 <= cu_count()) return 64;
        if (tiles256 <= cu_count()) return 128;
        *cols = kBlockN;
        return kBlockM;
    }
    return byte_tile_rows(fmt, m, n);
}

template <int F, int E>
static int launch_fmt(const GemmArgs& a, hipStream_t s) {
    int cols = 0, stages = 0;
    const int rows = tile_plan(F, E == EPI_F16_RES ? EPI_F16 : E, a.m, a.n, &cols, &stages);
    if constexpr (F == FMT_G128A8 || F == FMT_G128A16) {
        if constexpr (E != EPI_GLU && E != EPI_F8_24 && E != EPI_I8S) {
            if (k_split(F, E == EPI_F16_RES ? EPI_F16 : E, a.m, a.n, a.k) == 4) return launch_splitk<F, E, 4>(a, s);
        }
    }
    if constexpr (F == FMT_FP8 || F == FMT_I8 || F == FMT_G128A8 || F == FMT_G128A16) {
        if constexpr (E != EPI_GLU && E != EPI_F8_24 && E != EPI_I8S) {
            if (stages > 2) {
                if constexpr (F == FMT_G128A8) {
                    if (ring_occ2(F, a.m, a.n)) return launch_ring<F, E, 2, 2>(a, s);
                }
                if constexpr (F == FMT_G128A16) {
                    if (rows == 96) return launch_ring<F, E, 3>(a, s);
                }
                if constexpr (F == FMT_FP8 || F == FMT_I8) {
                    // two waves per SIMD (C1: 11.1 -> 10.0 us; FP8 750 x 1024 -> 4096: 10.9 -> 9.5)
                    if (rows == 64) return launch_ring8<F, E, 2>(a, s);
                    if (rows == 128) return launch_ring8<F, E, 4>(a, s);
                }
                return rows == 32 ? launch_ring<F, E, 1>(a, s) : (rows == 64 ? launch_ring<F, E, 2>(a, s) : launch_ring<F, E, 4>(a, s));
            }
        }
    }
    if constexpr (F == FMT_Q4K) {
        return launch_one<F, E>(a, s);
    } else if constexpr (F == FMT_F16 || F == FMT_G128A16) {
        if (cols == kBlockN) return launch_one<F, E>(a, s);
        return rows == 64 ? launch_two<F, E, 2>(a, s) : launch_two<F, E, 4>(a, s);
    } else {
        if (rows == 64) return launch_two<F, E, 2>(a, s);
        if (rows == 128) return launch_two<F, E, 4>(a, s);
        return launch_two<F, E, 8>(a, s);
    }
}

template <int F>
static int by_epi(int epi, const GemmArgs& a, hipStream_t s) {
    if constexpr (F == FMT_Q4K) {
        if (epi != EPI_F16 && epi != EPI_F32) {
            set_error("unsupported epilogue %d for format %d", epi, F);
            return -4;
        }
    }
    if constexpr (F == FMT_S4F6) {
        // the INT4 x INT4 FF2 expand (2:4 e4m3 out) and fp32 outputs (its exact sums)
        if (epi == EPI_F8_24) return launch_fmt<F, EPI_F8_24>(a, s);
        if (epi == EPI_F32) return launch_fmt<F, EPI_F32>(a, s);
        set_error("unsupported epilogue %d for format %d", epi, F);
        return -4;
    }
    switch (epi) {
    case EPI_F16: return a.residual ? launch_fmt<F, EPI_F16_RES>(a, s) : launch_fmt<F, EPI_F16>(a, s);
    case EPI_F32: return launch_fmt<F, EPI_F32>(a, s);
    case EPI_F8:
        if constexpr (F != FMT_Q4K) return launch_fmt<F, EPI_F8>(a, s);
        break;
    case EPI_F8_24:
        if constexpr (F != FMT_Q4K && F != FMT_G128F8) return launch_fmt<F, EPI_F8_24>(a, s);
        break;
    case EPI_I8S:
        // the byte-activation formats on the occupancy-2 engine
        if constexpr (F == FMT_FP8 || F == FMT_I8 || F == FMT_G128A8 || F == FMT_G128F8) return launch_fmt<F, EPI_I8S>(a, s);
        break;
    case EPI_I32:
        if constexpr (F == FMT_I8 || F == FMT_S4 || F == FMT_I8_SKIP) return launch_fmt<F, EPI_I32>(a, s);
        break;
    case EPI_GLU:
        // the paired value / gate weight rows need the 256-column tiles
        if constexpr (F == FMT_FP8) {
            if (a.n % 256 != 0 || a.ldo != a.n / 2 || !a.w_scales) {
                set_error("GLU needs n %% 256 == 0 weight rows, ldo == n/2 and weight scales");
                return -1;
            }
            return launch_one<F, EPI_GLU>(a, s);
        }
        break;
    default: break;
    }
    set_error("unsupported epilogue %d for format %d", epi, F);
    return -4;
}

static int k_step(int fmt) {
    switch (fmt) {
    case FMT_FP8: case FMT_I8: case FMT_G128A8: case FMT_I8_SKIP: case FMT_G128F8: case FMT_S4F6: return 128;
    case FMT_S4: case FMT_Q4K: return 256;
    default: return 64;
    }
}

int launch_gemm(int fmt, int epi, const GemmArgs& a, hipStream_t s) {
    if (a.m < 0 || a.n <= 0 || a.k <= 0) {
        set_error("invalid GEMM shape m=%d n=%d k=%d", a.m, a.n, a.k);
        return -1;
    }
    if ((fmt == FMT_G128A8 || fmt == FMT_G128A16 || fmt == FMT_G128F8) && a.k > 128 * kMaxG128Groups) {
        set_error("k=%d exceeds the %d groups of 128 the g128 kernels stage in LDS", a.k, kMaxG128Groups);
        return -1;
    }
    if (a.k % k_step(fmt) != 0 || ((fmt == FMT_G128A8 || fmt == FMT_G128A16 || fmt == FMT_G128F8) && a.k % 128 != 0)) {
        set_error("k=%d must be a multiple of %d for format %d", a.k, k_step(fmt), fmt);
        return -1;
    }
    if (a.n % 16 != 0 || a.ldo % 8 != 0 || (epi != EPI_GLU && (a.ldo % 16 != 0 || a.ldo < a.n))) {
        set_error("n=%d and ldo=%d must be multiples of 16 with ldo >= n", a.n, a.ldo);
        return -1;
    }
    // Operand loads address rows with 32-bit byte offsets from the base.
    if ((uint64_t)a.m * a.k * 2 > 0xffffffffull || (uint64_t)a.n * a.k * 2 > 0xffffffffull) {
        set_error("operands of m=%d n=%d k=%d exceed the 4 GiB a launch addresses", a.m, a.n, a.k);
        return -1;
    }
    if (((uintptr_t)a.a | (uintptr_t)a.b | (uintptr_t)a.out) & 15) {
        set_error("operand pointers must be 16-byte aligned");
        return -2;
    }
    // The epilogue reads residual rows, weight scales and biases as 16-byte vectors.
    if (((uintptr_t)a.residual | (uintptr_t)a.w_scales | (uintptr_t)a.bias) & 15) {
        set_error("residual, weight scale and bias pointers must be 16-byte aligned");
        return -2;
    }
    if (forced_tile_rows() < 0) {
        set_error("PK_GEMM_TILE_ROWS must be 64, 128 or 256");
        return -1;
    }
    if (a.m == 0) return 0;
    switch (fmt) {
    case FMT_FP8: return by_epi<FMT_FP8>(epi, a, s);
    case FMT_I8: return by_epi<FMT_I8>(epi, a, s);
    case FMT_S4: return by_epi<FMT_S4>(epi, a, s);
    case FMT_G128A8: return by_epi<FMT_G128A8>(epi, a, s);
    case FMT_F16: return by_epi<FMT_F16>(epi, a, s);
    case FMT_G128A16: return by_epi<FMT_G128A16>(epi, a, s);
    case FMT_I8_SKIP: return by_epi<FMT_I8_SKIP>(epi, a, s);
    case FMT_Q4K: return by_epi<FMT_Q4K>(epi, a, s);
    case FMT_G128F8: return by_epi<FMT_G128F8>(epi, a, s);
    case FMT_S4F6: return by_epi<FMT_S4F6>(epi, a, s);
    default: break;
    }
    set_error("unknown format %d", fmt);
    return -4;
}

int gemm_k_split(int fmt, int epi, int m, int n, int k) {
    if (fmt < FMT_FP8 || fmt > FMT_S4F6) return -4;
    if (forced_tile_rows() < 0) return -1;
    return k_split(fmt, epi == EPI_F16_RES ? EPI_F16 : epi, m, n, k);
}

int gemm_tile_plan(int fmt, int epi, int m, int n, int* cols, int* stages) {
    if (fmt < FMT_FP8 || fmt > FMT_S4F6) return -4;
    if (forced_tile_rows() < 0) return -1;
    return tile_plan(fmt, epi == EPI_F16_RES ? EPI_F16 : epi, m, n, cols, stages);
}

}  // namespace pk
