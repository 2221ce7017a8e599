// Batch-1 TDT joint (decoder.cu:690-759): per frame t,
//   score[o] = bias[o] + w_scale[o] * sum_k W[o,k] * relu(enc[t,k] + pred[k])
// then the greedy token / duration decision.  The GEMV is HBM/L2-bound: one
// wave64 per output row, each lane streaming 16 bytes (int8) or 16 bytes of
// fp16 per pass, the activation vector staged once per block in LDS.
#include <mutex>

#include "pk_kernels.hpp"

namespace pk {

template <bool kInt8>
__global__ __launch_bounds__(256) void joint_scores_kernel(const void* __restrict__ weight, const float* __restrict__ w_scales,
                                                           const float* __restrict__ bias, const uint16_t* __restrict__ enc,
                                                           const float* __restrict__ pred, float* __restrict__ scores,
                                                           int outputs, int hidden, int enc_stride) {
    __shared__ float x[1024];
    const int t = blockIdx.y;
    for (int k = threadIdx.x; k < hidden; k += 256)
        x[k] = __builtin_fmaxf(h2f(enc[(size_t)t * enc_stride + k]) + pred[k], 0.0f);
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= outputs) return;
    float sum = 0.0f;
    if constexpr (kInt8) {
        const int8_t* w = (const int8_t*)weight + (size_t)row * hidden;
        for (int k0 = lane * 16; k0 < hidden; k0 += 64 * 16) {
            const uint4 q = *(const uint4*)(w + k0);
            const uint32_t words[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int j = 0; j < 16; ++j)
                sum = __builtin_fmaf((float)(int8_t)(words[j >> 2] >> (8 * (j & 3))), x[k0 + j], sum);
        }
    } else {
        const uint16_t* w = (const uint16_t*)weight + (size_t)row * hidden;
        for (int k0 = lane * 8; k0 < hidden; k0 += 64 * 8) {
            const uint4 q = *(const uint4*)(w + k0);
            const uint32_t words[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int j = 0; j < 8; ++j)
                sum = __builtin_fmaf(h2f((uint16_t)(words[j >> 1] >> (16 * (j & 1)))), x[k0 + j], sum);
        }
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (lane == 0) {
        const float ws = kInt8 ? w_scales[row] : 1.0f;
        scores[(size_t)t * outputs + row] = __builtin_fmaf(ws, sum, bias ? bias[row] : 0.0f);
    }
}

// Streaming form for rows of a whole number of 128-byte lines (the model's
// 640-wide joint): a workgroup stages relu(enc[t] + pred) once and scores a
// run of `rows` consecutive rows.  A wave takes 8 rows at a time, 8 lanes per
// row; load u of lane p reads bytes [128u + 16p, +16) of its row, so each
// load instruction covers 8 whole lines, and NL = row bytes / 128 loads give
// the row.  Memory parallelism comes from many small resident workgroups
// (measured: 32 runs per CU with one row group in flight per wave streams a
// 344 MB matrix at 6.7 TB/s; deeper per-wave pipelines with fewer workgroups
// stayed below 6.2).  x is stored with 4 floats of skew per 64 (bank-distinct
// reads).  kNT marks the weight loads non-temporal, for matrices larger than
// the caches (one pass); a joint matrix that stays in L2 across frames is
// loaded normally.
template <bool kInt8, int NL, bool kNT>
__global__ __launch_bounds__(256) void joint_stream_kernel(const void* __restrict__ weight, const float* __restrict__ w_scales,
                                                           const float* __restrict__ bias, const uint16_t* __restrict__ enc,
                                                           const float* __restrict__ pred, float* __restrict__ scores,
                                                           int outputs, int enc_stride, int rows) {
    constexpr int kEl = kInt8 ? 16 : 8;           // elements per 16-byte load
    constexpr int kHidden = NL * (kInt8 ? 128 : 64);
    constexpr size_t kRowBytes = (size_t)NL * 128;
    __shared__ float x[kHidden + kHidden / 16];
    const int t = blockIdx.y;
    for (int k = threadIdx.x; k < kHidden; k += 256)
        x[k + 4 * (k >> 6)] = __builtin_fmaxf(h2f(enc[(size_t)t * enc_stride + k]) + pred[k], 0.0f);
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane >> 3, part = lane & 7;
    const int row0 = blockIdx.x * rows, row_end = min(row0 + rows, outputs);
    const uint8_t* wb = (const uint8_t*)weight + 16 * part;
    auto load = [&](uint4 (&q)[NL], int g) {
        const int r = min(g + sub, row_end - 1);
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
            const u32x4_t* src = (const u32x4_t*)(wb + (size_t)r * kRowBytes + 128 * u);
            const u32x4_t v = kNT ? __builtin_nontemporal_load(src) : *src;
            q[u] = uint4{v.x, v.y, v.z, v.w};
        }
    };
    auto dot = [&](const uint4 (&q)[NL]) -> float {
        float s = 0.0f;
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            const int k = u * (128 / (kInt8 ? 1 : 2)) + part * kEl;
            const float4* xv = (const float4*)(x + k + 4 * (k >> 6));
            const uint32_t wd[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
            for (int c = 0; c < kEl / 4; ++c) {
                const float4 xx = xv[c];
                const float xa[4] = {xx.x, xx.y, xx.z, xx.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int e = 4 * c + j;
                    const float w = kInt8 ? (float)(int8_t)(wd[e >> 2] >> (8 * (e & 3))) : h2f((uint16_t)(wd[e >> 1] >> (16 * (e & 1))));
                    s = __builtin_fmaf(w, xa[j], s);
                }
            }
        }
        // the 8 lanes of a row: quad swaps, then the other quad (DPP)
        s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0xb1, 0xf, 0xf, true));
        s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0x4e, 0xf, 0xf, true));
        return s + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0x141, 0xf, 0xf, true));
    };
    // The next group's loads are issued before this group's score store:
    // global stores count in vmcnt, so a wait for loads issued after a store
    // would also wait for the store.
    int g = row0 + 8 * wave;
    if (g >= row_end) return;
    uint4 q[NL];
    load(q, g);
    for (;;) {
        const float sum = dot(q);
        const int gn = g + 32;
        if (gn < row_end) load(q, gn);
        const int r = g + sub;
        if (part == 0 && r < row_end)
            scores[(size_t)t * outputs + r] = __builtin_fmaf(kInt8 ? w_scales[r] : 1.0f, sum, bias ? bias[r] : 0.0f);
        if (gn >= row_end) break;
        g = gn;
    }
}

// decoder.cu:34-46, 728-759: token = argmax over the first token_outputs
// scores, ties to the lower id; duration = first maximum of the next
// `durations` scores.
__global__ __launch_bounds__(256) void joint_decide_kernel(const float* __restrict__ scores, int* __restrict__ decision,
                                                           int outputs, int token_outputs, int durations) {
    __shared__ float best_s[4];
    __shared__ int best_i[4];
    const int t = blockIdx.x;
    const float* s = scores + (size_t)t * outputs;
    float bs = -__builtin_huge_valf();
    int bi = 0x7fffffff;
    for (int o = threadIdx.x; o < token_outputs; o += 256) {
        const float v = s[o];
        if (v > bs || (v == bs && o < bi)) { bs = v; bi = o; }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float os = __shfl_xor(bs, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (os > bs || (os == bs && oi < bi)) { bs = os; bi = oi; }
    }
    if ((threadIdx.x & 63) == 0) { best_s[threadIdx.x >> 6] = bs; best_i[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w)
            if (best_s[w] > bs || (best_s[w] == bs && best_i[w] < bi)) { bs = best_s[w]; bi = best_i[w]; }
        int d = 0;
        for (int i = 1; i < durations; ++i)
            if (s[token_outputs + i] > s[token_outputs + d]) d = i;
        decision[2 * t] = bi == 0x7fffffff ? 0 : bi;
        decision[2 * t + 1] = d;
    }
}

// ---- persistent blank scan (decoder.cu:690-783) ---------------------------------
//
// Between two emitted tokens the prediction vector is fixed, so the greedy TDT
// loop is a sequence of joint steps that only move the frame index, and the
// decision at a frame does not depend on how the scan got there.  One
// persistent launch runs those steps in rounds: every active workgroup keeps
// its slice of W in registers for the whole scan (8 rows per wave; lane l
// holds k = 2l + 128j, j < hidden/128) and, per round, scores its rows for the
// kScanRound frames frame, frame + 1, ... and publishes one 64-bit word per
// frame: its best token as an order-preserving key (score bits, then 0xffff -
// id), the duration decision when it owns the duration rows, and the round's
// tag.  The words are the grid barrier: each workgroup polls all of them
// (lane b reads workgroup b's words) until every tag is the current one, then
// takes the maximum per frame, and every thread applies the greedy rules over
// the round's decisions, identically, until a non-blank token (the prediction
// network must run before the next step), the frames run out, or the frame
// leaves the round.  A barrier costs a memory round trip through the device-
// coherent level; a round amortises it over the steps its frames cover.  The
// encoder rows come from a window of kScanWin frames each workgroup keeps in
// LDS, refilled when the round would leave it.
//
// Logical row i of the scan is joint row T + i for i < D (the durations, all
// in workgroup 0's wave 0) and row i - D for the tokens.  Workgroups are
// dispatched round-robin over the 8 XCDs; only those with blockIdx % 8 == 0
// work, so the active ones share one XCD's L2.

constexpr int kScanRows = 8;      // joint rows per wave
constexpr int kScanRound = 8;     // frames scored per round
constexpr int kScanWin = 32;      // encoder frames in the LDS window (32 x hidden x 2 bytes <= 64 KiB)
constexpr int kScanMaxBlocks = 64;
constexpr uint32_t kScanSpinLimit = 1u << 22;
static_assert(8 + 2 * 2 * kScanRound * kScanMaxBlocks <= kJointScanWorkspaceWords, "scan words fit the workspace");

struct ScanArgs {
    const void* w;
    const float* w_scales;
    const float* bias;
    const uint16_t* enc;
    const float* pred;
    int* state;
    uint32_t* ws;  // [0] abort flag; words 8.. : u64 [2 parities][kScanRound frames][kScanMaxBlocks]
    int outputs, hidden, token_outputs, durations, frames, enc_stride, max_symbols;
};

__device__ __forceinline__ uint32_t ordered_bits(float score) {
    if (score == 0.0f) score = 0.0f;  // -0 and +0 tie on the id
    const uint32_t bits = __float_as_uint(score);
    return (bits & 0x80000000u) ? ~bits : (bits ^ 0x80000000u);
}

// KP = hidden / 128 pairs of k per lane.  At most 256 VGPRs (two workgroups
// per CU): the up to 64 active workgroups must all be resident on the 32 CUs
// of one XCD, or the first round's barrier never completes.
template <bool kInt8, int KP>
__global__ __launch_bounds__(256, 2) void joint_scan_kernel(ScanArgs p) {
    if (blockIdx.x & 7) return;
    __shared__ unsigned long long wave_key[4][kScanRound];
    __shared__ int dur_s[kScanRound];
    __shared__ int dec_tok[kScanRound], dec_dur[kScanRound];
    const int blk = blockIdx.x >> 3;
    const int nblocks = gridDim.x >> 3;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int T = p.token_outputs, D = p.durations;
    unsigned long long* const words = (unsigned long long*)(p.ws + 8);
    const bool watcher = lane < nblocks;

    uint32_t w[kScanRows][KP];
    float wsc[kScanRows], wb[kScanRows];
    int rid[kScanRows];
#pragma unroll
    for (int r = 0; r < kScanRows; ++r) {
        const int i = (blk * 4 + wave) * kScanRows + r;
        rid[r] = i < D ? T + i : (i < T + D ? i - D : -1);
        const int row = rid[r] < 0 ? p.outputs - 1 : rid[r];
#pragma unroll
        for (int j = 0; j < KP; ++j) {
            const int k = 2 * lane + 128 * j;
            if constexpr (kInt8) w[r][j] = *(const uint16_t*)((const int8_t*)p.w + (size_t)row * p.hidden + k);
            else w[r][j] = *(const uint32_t*)((const uint16_t*)p.w + (size_t)row * p.hidden + k);
        }
        wsc[r] = kInt8 ? p.w_scales[row] : 1.0f;
        wb[r] = p.bias ? p.bias[row] : 0.0f;
    }
    float pv[2 * KP];
#pragma unroll
    for (int j = 0; j < KP; ++j) {
        pv[2 * j] = p.pred[2 * lane + 128 * j];
        pv[2 * j + 1] = p.pred[2 * lane + 128 * j + 1];
    }
    // encoder window: frames [win_base, win_base + kScanWin) as fp16 pairs
    extern __shared__ uint32_t enc_win[];
    constexpr int kPairs = 64 * KP;  // hidden / 2
    int win_base = 0;
    auto load_win = [&](int base) {
        for (int i = threadIdx.x; i < kScanWin * kPairs; i += 256) {
            const int f = base + i / kPairs;
            enc_win[i] = f < p.frames ? *(const uint32_t*)(p.enc + (size_t)f * p.enc_stride + 2 * (i % kPairs)) : 0u;
        }
        win_base = base;
        __syncthreads();
    };

    int frame = p.state[0], symbols = p.state[1];
    int token = -1, steps = 0, rounds = 0;
    bool failed = false, done = false;
    const int blank = T - 1;
    if (frame < p.frames) load_win(frame);

    while (frame < p.frames && !done) {
        // every workgroup takes the same decisions, so the refill is uniform
        if (frame + kScanRound > win_base + kScanWin) load_win(frame);
        const int f0 = frame;
        // per round frame: this wave's 8 row scores, reduced over the lanes,
        // then the wave's best token (and, in workgroup 0's wave 0, the
        // duration) into LDS
#pragma unroll 1
        for (int c = 0; c < kScanRound; ++c) {
            const int f = min(f0 + c, p.frames - 1) - win_base;
            float x[2 * KP];
#pragma unroll
            for (int j = 0; j < KP; ++j) {
                const uint32_t ev = enc_win[f * kPairs + lane + 64 * j];
                x[2 * j] = __builtin_fmaxf(h2f((uint16_t)(ev & 0xffffu)) + pv[2 * j], 0.0f);
                x[2 * j + 1] = __builtin_fmaxf(h2f((uint16_t)(ev >> 16)) + pv[2 * j + 1], 0.0f);
            }
            float acc[kScanRows];
#pragma unroll
            for (int r = 0; r < kScanRows; ++r) {
                float sum = 0.0f;
#pragma unroll
                for (int j = 0; j < KP; ++j) {
                    float w0, w1;
                    if constexpr (kInt8) {
                        w0 = (float)(int8_t)(w[r][j] & 0xffu);
                        w1 = (float)(int8_t)((w[r][j] >> 8) & 0xffu);
                    } else {
                        w0 = h2f((uint16_t)(w[r][j] & 0xffffu));
                        w1 = h2f((uint16_t)(w[r][j] >> 16));
                    }
                    sum = __builtin_fmaf(w0, x[2 * j], sum);
                    sum = __builtin_fmaf(w1, x[2 * j + 1], sum);
                }
                acc[r] = sum;
            }
#pragma unroll
            for (int off = 1; off < 64; off <<= 1)
#pragma unroll
                for (int r = 0; r < kScanRows; ++r) acc[r] = add_level(acc[r], off);
            float bs = -__builtin_huge_valf(), dbest = 0.0f;
            int bi = 0x7fffffff, dur = 0;
#pragma unroll
            for (int r = 0; r < kScanRows; ++r) {
                const float score = __builtin_fmaf(wsc[r], acc[r], wb[r]);
                const int id = rid[r];
                if (id >= T) {  // duration id - T, first maximum wins
                    if (id == T || score > dbest) { dbest = score; dur = id - T; }
                } else if (id >= 0) {
                    if (score > bs || (score == bs && id < bi)) { bs = score; bi = id; }
                }
            }
            if (lane == 0) {
                wave_key[wave][c] = bi == 0x7fffffff ? 0ull
                                                     : (((unsigned long long)ordered_bits(bs) << 32) |
                                                        ((unsigned long long)(0xffffu - (uint32_t)bi) << 16));
                if (blk == 0 && wave == 0) dur_s[c] = dur;
            }
        }
        __syncthreads();
        const int par = (rounds & 1) * kScanRound * kScanMaxBlocks;
        const uint32_t tag = (uint32_t)(rounds + 1) & 0x1fffu;
        // thread c publishes this workgroup's word for round frame c
        if (threadIdx.x < kScanRound) {
            const int c = threadIdx.x;
            unsigned long long key = wave_key[0][c];
            for (int i = 1; i < 4; ++i) key = wave_key[i][c] > key ? wave_key[i][c] : key;
            key |= (unsigned long long)((uint32_t)(blk == 0 ? dur_s[c] : 0) << 13) | tag;
            __hip_atomic_store(words + par + c * kScanMaxBlocks + blk, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // poll: lane b of every wave reads workgroup b's words; wave w reduces
        // frames w and w + 4
        unsigned long long got[2] = {0ull, 0ull};
        uint32_t spins = 0;
        while (true) {
            bool ready = true;
            if (watcher) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    got[h] = __hip_atomic_load(words + par + (wave + 4 * h) * kScanMaxBlocks + lane, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                    ready = ready && ((uint32_t)got[h] & 0x1fffu) == tag;
                }
            }
            if (__builtin_amdgcn_ballot_w64(!ready) == 0) break;
            if ((++spins & 63) == 0 &&
                (spins > kScanSpinLimit || __hip_atomic_load(&p.ws[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)) {
                __hip_atomic_store(&p.ws[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                failed = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        // a wave that gave up stops the workgroup (the flag makes every other
        // workgroup's poll give up too)
        if (__syncthreads_or(failed)) {
            failed = true;
            break;
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // workgroup 0's word carries the duration; the maximum word the token
            const int dur = (int)(((uint32_t)__shfl(got[h], 0, 64) >> 13) & 7u);
            unsigned long long best = watcher ? got[h] : 0ull;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) best = max_level(best, off);
            if (lane == 0) {
                dec_tok[wave + 4 * h] = (int)(0xffffu - (((uint32_t)best) >> 16));
                dec_dur[wave + 4 * h] = dur;
            }
        }
        __syncthreads();
        ++rounds;
        // the greedy rules (decoder.cu:773-783) over the round's decisions, in
        // every thread alike
        while (true) {
            const int c = frame - f0;
            token = dec_tok[c];
            const int dur = dec_dur[c];
            ++steps;
            ++symbols;
            frame += dur;
            if (dur != 0 || symbols == p.max_symbols) {
                if (dur == 0) ++frame;
                symbols = 0;
            }
            if (token != blank) {
                done = true;
                break;
            }
            token = -1;
            if (frame >= p.frames || frame - f0 >= kScanRound) break;
        }
        // the LDS decision and key slots are rewritten next round
        __syncthreads();
    }
    if (blk == 0 && threadIdx.x == 0) {
        p.state[0] = frame;
        p.state[1] = symbols;
        p.state[2] = failed ? -2 : token;
        p.state[3] = steps;
    }
}

__global__ void scan_clear_kernel(uint32_t* ws) {
    for (int i = threadIdx.x; i < kJointScanWorkspaceWords; i += blockDim.x) ws[i] = 0u;
}

int launch_joint_scan(const void* w, int w_int8, const float* w_scales, const float* bias, const uint16_t* enc, const float* pred,
                      int outputs, int hidden, int token_outputs, int durations, int frames, int enc_stride, int max_symbols,
                      int* state, uint32_t* workspace, hipStream_t s) {
    const int active = (token_outputs + durations + 4 * kScanRows - 1) / (4 * kScanRows);
    ScanArgs a{w, w_scales, bias, enc, pred, state, workspace, outputs, hidden, token_outputs, durations, frames, enc_stride, max_symbols};
    scan_clear_kernel<<<1, 256, 0, s>>>(workspace);
    const dim3 grid(8 * active);
    const size_t win = (size_t)kScanWin * (hidden / 2) * sizeof(uint32_t);
    switch (hidden >> 7) {
#define PK_SCAN_CASE(KP)                                                              \
    case KP:                                                                          \
        if (w_int8) joint_scan_kernel<true, KP><<<grid, 256, win, s>>>(a);           \
        else joint_scan_kernel<false, KP><<<grid, 256, win, s>>>(a);                 \
        break;
        PK_SCAN_CASE(1) PK_SCAN_CASE(2) PK_SCAN_CASE(3) PK_SCAN_CASE(4)
        PK_SCAN_CASE(5) PK_SCAN_CASE(6) PK_SCAN_CASE(7) PK_SCAN_CASE(8)
#undef PK_SCAN_CASE
    default: break;
    }
    return 0;
}

// ---- the same scan with library-owned scratch (no allocation) ---------------
//
// The scan's workspace (abort flag + 2 x 64 published words, 512 words) in a
// file-scope device array: each GPU the library runs on holds its own copy
// until the process ends.  Host code never passes the array's name to a
// kernel (on the host it is only a stand-in for the symbol): the device
// address of each GPU's copy is looked up once per device with
// hipGetSymbolAddress, with that device current, and kept.  Every call on a
// GPU shares that GPU's copy; launch_joint_scan clears it with a fill kernel
// before the scan kernel, so calls on one stream are independent, and calls
// that overlap on one GPU (different streams) race on it.
static __device__ __align__(256) uint32_t scratch[kJointScanWorkspaceWords];

namespace {
constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
uint32_t* scratch_ptr[kMaxDevices] = {};
}  // namespace

int joint_scan_scratch(uint32_t** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error("hipGetDevice failed: %s", hipGetErrorString(e));
        return -3;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        set_error("device %d beyond the %d devices the static scan scratch tracks", dev, kMaxDevices);
        return -4;
    }
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            set_error("hipGetSymbolAddress(scan scratch) failed: %s", hipGetErrorString(e));
            return -3;
        }
        scratch_ptr[dev] = (uint32_t*)ptr;
    }
    *out = scratch_ptr[dev];
    return 0;
}

int launch_joint(const void* w, int w_int8, const float* w_scales, const float* bias, const void* enc, const float* pred,
                 float* scores, int* decision, int outputs, int hidden, int token_outputs, int durations, int steps,
                 int enc_stride, hipStream_t s) {
    if (steps == 0) return 0;
    const int nl = w_int8 ? hidden / 128 : hidden / 64;
    if ((w_int8 ? hidden % 128 : hidden % 64) == 0 && nl >= 1 && nl <= 16) {
        // Rows per workgroup: 32 for the model's 1030-row joint (enough
        // workgroups for one frame); a large matrix is split into about 32
        // runs per CU.
        const int per = 32 * max(1, (outputs + 32 * 32 * cu_count() - 1) / (32 * 32 * cu_count()));
        const dim3 grid((outputs + per - 1) / per, steps);
        const bool nt = (size_t)outputs * hidden * (w_int8 ? 1 : 2) > ((size_t)128 << 20);
        switch (nl + (w_int8 ? 0 : 100)) {
#define PK_JS(I8, N)                                                                                                       \
    case N + (I8 ? 0 : 100):                                                                                               \
        if (nt)                                                                                                            \
            joint_stream_kernel<I8, N, true><<<grid, 256, 0, s>>>(w, w_scales, bias, (const uint16_t*)enc, pred, scores,   \
                                                                  outputs, enc_stride, per);                               \
        else                                                                                                               \
            joint_stream_kernel<I8, N, false><<<grid, 256, 0, s>>>(w, w_scales, bias, (const uint16_t*)enc, pred, scores,  \
                                                                   outputs, enc_stride, per);                              \
        break;
            PK_JS(true, 1) PK_JS(true, 2) PK_JS(true, 3) PK_JS(true, 4) PK_JS(true, 5) PK_JS(true, 6) PK_JS(true, 7) PK_JS(true, 8)
            PK_JS(false, 2) PK_JS(false, 4) PK_JS(false, 6) PK_JS(false, 8) PK_JS(false, 10) PK_JS(false, 12) PK_JS(false, 14)
            PK_JS(false, 16)
#undef PK_JS
            default: goto generic;
        }
        if (decision) joint_decide_kernel<<<steps, 256, 0, s>>>(scores, decision, outputs, token_outputs, durations);
        return 0;
    }
generic:
    const dim3 grid((outputs + 3) / 4, steps);
    if (w_int8)
        joint_scores_kernel<true><<<grid, 256, 0, s>>>(w, w_scales, bias, (const uint16_t*)enc, pred, scores, outputs, hidden, enc_stride);
    else
        joint_scores_kernel<false><<<grid, 256, 0, s>>>(w, w_scales, bias, (const uint16_t*)enc, pred, scores, outputs, hidden, enc_stride);
    if (decision) joint_decide_kernel<<<steps, 256, 0, s>>>(scores, decision, outputs, token_outputs, durations);
    return 0;
}

}  // namespace pk
