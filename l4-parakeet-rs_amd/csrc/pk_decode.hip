// Batch-1 greedy TDT decode in one persistent launch: 2-layer LSTM prediction
// network (gate rows i, f, g, o of 4H), projection + bias, joint, token /
// duration decision and the frame / symbol rules, for all frames of one
// utterance.  Two prediction-network forms, as in the reference:
//  - fp16 (decoder.cu:146-445, tdt_persistent_fp16): fp16 weights, fp32 state;
//  - long (decoder.cu:452-784, tdt_persistent_fp8, used for utterances of
//    1024 frames and more, decoder.rs:15,86-92): W_hh of both layers and W_ih
//    of layer 1 as per-tensor symmetric INT8 derived inside the launch
//    (scale = max|w| / 127), hidden states carried as INT8 at a fixed 1/127
//    scale next to the fp32 ones, layer 0's input terms read from a
//    [tokens x 4H] fp16 table (embedding x W_ih0^T), and the recurrent terms of
//    the state the next update consumes summed as soon as that state exists.
//
// Every weight stays in registers for the whole decode: the grid is one
// workgroup per CU (up to 256, 4 wave64 each) and wave w owns LSTM hidden unit
// w of both layers (4 gates x (W_ih, W_hh) rows), projection row w and joint
// rows 2w, 2w+1 (logical order: the duration rows first, so workgroup 0 holds
// them all).  Lane l holds k = 2l + 128j (j < H/128) of every row it owns.
// The phases (layer 0, layer 1, projection, joint) are separated by a grid
// barrier made of per-workgroup published 64-bit words (a step tag and, for
// the joint, the workgroup's best token key and workgroup 0's duration): every
// workgroup polls all words in parallel, so one barrier costs about one memory
// round trip, and the joint's decision comes with its barrier.  State vectors
// (h, c of both layers, double buffered as committed / candidate, and the
// prediction) move through agent-scope atomic stores and loads in a caller
// workspace.  Blank steps run only the joint; an emitted token commits the
// candidate state and re-runs the prediction network on its embedding.
//
// Long form: lane l holds bytes 4l + 256j (j < ceil(H/256)) of every INT8
// row; a gate's INT8 dot product is summed exactly as an integer over the
// wave (|sum| <= H * 127 * 127 < 2^24), converted once and scaled by
// scale / 127.  Layer 0 needs no weights of its own once its recurrent sums
// are known (its input terms are table rows), so every workgroup evaluates all
// of its units as soon as the token is decided and goes straight on to layer
// 1: an update costs two grid barriers (after layer 1, after the projection),
// not three.  The recurrent sums of a candidate state are taken as soon as
// that state exists (layer 0's next to layer 1, layer 1's in the projection
// phase) and used by the update after a token commits it.  Layer 1's cell
// state stays in the owning wave's registers, layer 0's in every thread that
// evaluates the unit; the INT8 layer-1 banks, the candidate fp32 layer-1
// output, the layer-0 sums and the prediction go through the workspace.
#include "pk_kernels.hpp"

namespace pk {

namespace {

constexpr int kDecThreads = 256;
constexpr int kDecMaxBlocks = 256;
constexpr uint32_t kDecSpinLimit = 1u << 22;
constexpr int kDecWords = 8;                                // u32 offset of the barrier words
constexpr int kDecState = kDecWords + 2 * kDecMaxBlocks * 2;  // u32 offset of the state vectors, after the words
static_assert(kDecState == 1032, "workspace layout");
// Frames a joint round scores against one prediction (its window), and the
// words of the joint rounds' barrier: per workgroup one key per window frame,
// each carrying the barrier tag (2 epoch slots x kWin x 256 u64, word-major so
// that the poll reads consecutive words), after the state vectors.
constexpr int kWin = 8;
constexpr int kDecExtWords = 2 * kDecMaxBlocks * kWin * 2;

struct DecodeArgs {
    const uint16_t* enc;    // [frames x enc_stride] fp16
    const uint16_t* emb;    // [token_outputs - 1 x H] fp16 (fp16 form)
    const uint16_t* table;  // [token_outputs - 1 x 4H] fp16 layer-0 input terms (long form)
    const uint16_t* w_ih[2];
    const uint16_t* w_hh[2];
    const float* b_ih[2];
    const float* b_hh[2];
    const uint16_t* w_proj;
    const float* b_proj;
    const void* w_joint;  // fp16 or int8 [outputs x H]
    const float* joint_scales;
    const float* b_joint;
    int32_t* tokens;
    int32_t* result;  // {tokens emitted, final frame, status, joint steps}
    uint32_t* ws;     // [0] abort; words at kDecWords (2 x 256 u64 = 1024 u32); state floats at kDecState
    int frames, enc_stride, outputs, token_outputs, durations, max_symbols, capacity;
};

__device__ __forceinline__ uint32_t key_bits(float score) {
    if (score == 0.0f) score = 0.0f;
    const uint32_t bits = __float_as_uint(score);
    return (bits & 0x80000000u) ? ~bits : (bits ^ 0x80000000u);
}

__device__ __forceinline__ float sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

__device__ __forceinline__ float2 ld2(const float* p) {
    const unsigned long long v = __hip_atomic_load((const unsigned long long*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
}
__device__ __forceinline__ float ld1(const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st1(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = add_level(v, off);
    return v;
}
__device__ __forceinline__ int wave_isum(int v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = add_level(v, off);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = max_level(v, off);
    return v;
}

// decoder.cu:95-97 quantize_i8: round to nearest even, clamp to +-127.
__device__ __forceinline__ int quant_i8(float v) { return max(-127, min(127, (int)__builtin_rintf(v))); }

// exp(x) from IEEE basic operations only, so that the long form's cell (whose
// outputs are rounded to INT8) is reproduced bit for bit by a CPU evaluating
// the same operations: Cody-Waite reduction x = n ln2 + r (ln2 split into a
// 16-bit head, so n * head is exact, and a tail), e^r by its degree-7 Taylor
// polynomial (|r| <= 0.347: truncation error 5e-9 relative), times 2^n.
// Within 0.82 ulp of exp over [-87, 88]; expf / tanhf of the reference are
// within about an ulp too.
__device__ __forceinline__ float det_exp(float x) {
    if (x != x) return x;
    x = __builtin_fminf(__builtin_fmaxf(x, -104.0f), 89.0f);
    const float n = __builtin_rintf(x * 1.44269504f);
    float r = __builtin_fmaf(n, -0.693145751953125f, x);
    r = __builtin_fmaf(n, -1.428606765330187e-06f, r);
    float q = 1.98412698e-04f;
    q = __builtin_fmaf(q, r, 1.38888889e-03f);
    q = __builtin_fmaf(q, r, 8.33333333e-03f);
    q = __builtin_fmaf(q, r, 4.16666667e-02f);
    q = __builtin_fmaf(q, r, 1.66666667e-01f);
    q = __builtin_fmaf(q, r, 0.5f);
    q = __builtin_fmaf(q, r, 1.0f);
    q = __builtin_fmaf(q, r, 1.0f);
    return __builtin_ldexpf(q, (int)n);
}
__device__ __forceinline__ float det_sigmoid(float v) { return 1.0f / (1.0f + det_exp(-v)); }
// tanh(x) = sign(x) (1 - e^-2|x|) / (1 + e^-2|x|): absolute error ~1e-7.
__device__ __forceinline__ float det_tanh(float v) {
    const float t = det_exp(-2.0f * __builtin_fabsf(v));
    return __builtin_copysignf((1.0f - t) / (1.0f + t), v);
}

// decoder.cu:116-129 lstm_cell with the transcendental functions above; the
// cell update is fma(f, c, i * g).
__device__ __forceinline__ void lstm_cell(const float (&s)[4], float c_prev, float& c_out, float& h_out) {
    const float ig = det_sigmoid(s[0]), fg = det_sigmoid(s[1]), cg = det_tanh(s[2]), og = det_sigmoid(s[3]);
    c_out = __builtin_fmaf(fg, c_prev, ig * cg);
    h_out = og * det_tanh(c_out);
}

__device__ __forceinline__ uint32_t ld_word(const uint32_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_word(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// fp16 pair -> two floats
__device__ __forceinline__ float lo16(uint32_t w) { return h2f((uint16_t)(w & 0xffffu)); }
__device__ __forceinline__ float hi16(uint32_t w) { return h2f((uint16_t)(w >> 16)); }

template <bool kInt8, int KP, bool kLong>
__global__ __launch_bounds__(kDecThreads, 1) void tdt_decode_kernel(DecodeArgs p) {
    constexpr int H = 128 * KP;
    constexpr int KD = (KP + 1) / 2;  // INT8 dwords per lane and row (long form)
    __shared__ float red_s[12];
    __shared__ uint32_t qb_s[4];
    __shared__ float dur_sc[kWin][8];
    __shared__ unsigned long long win_w[4][kWin];  // per wave, then the decided key per window frame
    __shared__ int win_tok[kWin], win_dur[kWin];
    __shared__ int stop_s;
    // long form: the new INT8 layer-0 output, computed whole by every workgroup
    __shared__ uint32_t q0_s[kLong ? H / 4 : 1];
    const int blk = blockIdx.x, nblocks = gridDim.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int gw = blk * 4 + wave;
    const int T = p.token_outputs, D = p.durations, blank = T - 1;
    unsigned long long* words = (unsigned long long*)(p.ws + kDecWords);
    float* st = (float*)(p.ws + kDecState);
    // state: h[buf][layer][H], c[buf][layer][H], pred[H]
    auto hp = [&](int buf, int layer) { return st + (buf * 2 + layer) * H; };
    auto cp = [&](int buf, int layer) { return st + 4 * H + (buf * 2 + layer) * H; };
    float* pred = st + 8 * H;
    // long form: INT8 hidden vectors [bank][layer][H] bytes, candidate fp32
    // layer-1 output, per-workgroup weight maxima [blocks][3]
    uint32_t* qh = p.ws + kDecState;
    auto qbank = [&](int bank, int layer) { return qh + (bank * 2 + layer) * (H / 4); };
    float* h1c = st + H;
    float* maxima = st + 2 * H;

    // Encoder rows of a joint round's window (frames pf_base .. pf_base +
    // kWin - 1): loaded during the first barrier of a prediction update, when
    // the next round's frame is known, or directly by a round whose window
    // they are not.  pf_base = frame of candidate 0 (-1: none).
    uint32_t cand[kWin][KP];
    int pf_base = -1;
    bool do_pf = false;
    auto prefetch = [&]() {
#pragma unroll
        for (int d = 0; d < kWin; ++d) {
            const int f = pf_base + d;
            const bool ok = f < p.frames;
            const uint16_t* e = p.enc + (size_t)(ok ? f : 0) * p.enc_stride + 2 * lane;
#pragma unroll
            for (int j = 0; j < KP; ++j) cand[d][j] = ok ? *(const uint32_t*)(e + 128 * j) : 0u;
        }
    };

    // ---- grid barrier: publish this workgroup's word, wait for every tag ---------
    uint32_t epoch = 0;
    bool failed = false;
    auto barrier = [&](unsigned long long payload) -> unsigned long long {
        // this wave's state stores have completed before the word goes out
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const uint32_t tag = (epoch + 1) & 0x1fffu;
        unsigned long long* slot = words + (epoch & 1) * kDecMaxBlocks;
        if (tid == 0) __hip_atomic_store(slot + blk, payload | tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (do_pf) prefetch();  // in flight during the poll
        do_pf = false;
        unsigned long long mine = 0;
        uint32_t spins = 0;
        while (true) {
            bool ready = true;
            if (tid < nblocks) {
                mine = __hip_atomic_load(slot + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ready = ((uint32_t)mine & 0x1fffu) == tag;
            }
            if (__syncthreads_and(ready)) break;
            if ((++spins & 63) == 0) {
                // one thread decides, so the whole workgroup leaves together
                if (tid == 0)
                    stop_s = spins > kDecSpinLimit || __hip_atomic_load(&p.ws[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
                __syncthreads();
                if (stop_s) {
                    if (tid == 0) __hip_atomic_store(&p.ws[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    failed = true;
                    break;
                }
            }
            __builtin_amdgcn_s_sleep(1);
        }
        ++epoch;
        return mine;  // thread t holds workgroup t's word
    };
    // The joint rounds' barrier: thread c < kWin publishes this workgroup's key
    // for window frame c, each key tagged, so all go out together and the poll
    // itself gathers every workgroup's keys (thread t: workgroup t's, in got).
    // word-major ([parity][frame][workgroup]): the poll's lanes read consecutive words
    unsigned long long* wwords = (unsigned long long*)(p.ws + kDecState + 9 * H);  // [2][kWin][256]
    auto barrier_win = [&](unsigned long long key, unsigned long long (&got)[kWin]) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const uint32_t tag = (epoch + 1) & 0x1fffu;
        unsigned long long* slot = wwords + (size_t)(epoch & 1) * kDecMaxBlocks * kWin;
        if (tid < kWin) __hip_atomic_store(slot + tid * kDecMaxBlocks + blk, key | tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (do_pf) prefetch();
        do_pf = false;
        uint32_t spins = 0;
#pragma unroll
        for (int c = 0; c < kWin; ++c) got[c] = 0ull;
        while (true) {
            bool ready = true;
            if (tid < nblocks) {
#pragma unroll
                for (int c = 0; c < kWin; ++c) {
                    got[c] = __hip_atomic_load(slot + c * kDecMaxBlocks + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ready = ready && ((uint32_t)got[c] & 0x1fffu) == tag;
                }
            }
            if (__syncthreads_and(ready)) break;
            if ((++spins & 63) == 0) {
                if (tid == 0)
                    stop_s = spins > kDecSpinLimit || __hip_atomic_load(&p.ws[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
                __syncthreads();
                if (stop_s) {
                    if (tid == 0) __hip_atomic_store(&p.ws[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    failed = true;
                    break;
                }
            }
            __builtin_amdgcn_s_sleep(1);
        }
        ++epoch;
    };

    // long form: layer-0 recurrent sums of the candidate state [bank][H][4 gates]
    // (the committed bank is the other), published by the unit's owner
    int32_t* rs0w = (int32_t*)(p.ws + kDecState + 9 * H + kDecExtWords);

    // ---- weights into registers --------------------------------------------------
    const bool owns_unit = gw < H;
    const int u = owns_unit ? gw : 0;
    uint32_t wih[kLong ? 1 : 2][4][KP], whh[kLong ? 1 : 2][4][KP], wpj[KP];
    // long form: INT8 rows of W_hh0, W_hh1, W_ih1 and their scale / 127
    uint32_t qw[kLong ? 3 : 1][4][KD];
    float cq[3] = {1.0f, 1.0f, 1.0f};
    float bias[2][4];
#pragma unroll
    for (int l = 0; l < 2; ++l)
#pragma unroll
        for (int g = 0; g < 4; ++g) bias[l][g] = p.b_ih[l][g * H + u] + p.b_hh[l][g * H + u];
    if constexpr (!kLong) {
#pragma unroll
        for (int l = 0; l < 2; ++l)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const size_t row = (size_t)(g * H + u) * H;
#pragma unroll
                for (int j = 0; j < KP; ++j) {
                    const int k = 2 * lane + 128 * j;
                    wih[l][g][j] = *(const uint32_t*)(p.w_ih[l] + row + k);
                    whh[l][g][j] = *(const uint32_t*)(p.w_hh[l] + row + k);
                }
            }
    } else {
        // decoder.cu:520-575: per-tensor maxima over the whole grid, scale =
        // max / 127 (1 for an all-zero matrix), q = quantize_i8(w / scale).
        const uint16_t* src[3] = {p.w_hh[0], p.w_hh[1], p.w_ih[1]};
        const size_t n8 = (size_t)H * H / 2;  // 16-byte chunks of a [4H x H] fp16 matrix
        const size_t gt = (size_t)blk * kDecThreads + tid, gs = (size_t)nblocks * kDecThreads;
        float mx[3];
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            float a = 0.0f;
            for (size_t i = gt; i < n8; i += gs) {
                const uint4 v = ((const uint4*)src[m])[i];
                const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    a = __builtin_fmaxf(a, __builtin_fmaxf(__builtin_fabsf(lo16(w4[e])), __builtin_fabsf(hi16(w4[e]))));
            }
            mx[m] = wave_max(a);
        }
        if (lane == 0)
#pragma unroll
            for (int m = 0; m < 3; ++m) red_s[wave * 3 + m] = mx[m];
        __syncthreads();
        if (tid == 0)
#pragma unroll
            for (int m = 0; m < 3; ++m)
                st1(maxima + blk * 3 + m, __builtin_fmaxf(__builtin_fmaxf(red_s[m], red_s[3 + m]), __builtin_fmaxf(red_s[6 + m], red_s[9 + m])));
        barrier(0);
        float r[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            if (tid < nblocks) r[m] = ld1(maxima + tid * 3 + m);
            r[m] = wave_max(r[m]);
        }
        if (lane == 0)
#pragma unroll
            for (int m = 0; m < 3; ++m) red_s[wave * 3 + m] = r[m];
        __syncthreads();
        float scale[3];
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            const float t = __builtin_fmaxf(__builtin_fmaxf(red_s[m], red_s[3 + m]), __builtin_fmaxf(red_s[6 + m], red_s[9 + m]));
            scale[m] = t > 0.0f ? t / 127.0f : 1.0f;
            cq[m] = scale[m] / 127.0f;
        }
#pragma unroll
        for (int m = 0; m < 3; ++m)
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int j = 0; j < KD; ++j) {
                    const int k = 4 * lane + 256 * j;
                    uint32_t word = 0;
                    if (k < H) {
                        const uint2 hv = *(const uint2*)(src[m] + (size_t)(g * H + u) * H + k);
                        word = (uint32_t)(uint8_t)quant_i8(lo16(hv.x) / scale[m]) | ((uint32_t)(uint8_t)quant_i8(hi16(hv.x) / scale[m]) << 8) |
                               ((uint32_t)(uint8_t)quant_i8(lo16(hv.y) / scale[m]) << 16) |
                               ((uint32_t)(uint8_t)quant_i8(hi16(hv.y) / scale[m]) << 24);
                    }
                    qw[m][g][j] = word;
                }
    }
#pragma unroll
    for (int j = 0; j < KP; ++j) wpj[j] = *(const uint32_t*)(p.w_proj + (size_t)u * H + 2 * lane + 128 * j);
    const float bpj = p.b_proj[u];
    uint32_t wj[2][KP];
    float wjs[2], wjb[2];
    int jid[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int i = 2 * gw + r;
        jid[r] = i < D ? T + i : (i < T + D ? i - D : -1);
        const int row = jid[r] < 0 ? p.outputs - 1 : jid[r];
#pragma unroll
        for (int j = 0; j < KP; ++j) {
            const int k = 2 * lane + 128 * j;
            if constexpr (kInt8) wj[r][j] = *(const uint16_t*)((const int8_t*)p.w_joint + (size_t)row * H + k);
            else wj[r][j] = *(const uint32_t*)((const uint16_t*)p.w_joint + (size_t)row * H + k);
        }
        wjs[r] = kInt8 ? p.joint_scales[row] : 1.0f;
        wjb[r] = p.b_joint[row];
    }

    // long form: layer 0 of every unit tid + 256 i is evaluated by this thread in
    // every workgroup (identical operations, so identical values everywhere):
    // its bias, committed / candidate cell state and the recurrent sums of the
    // state the next update consumes
    constexpr int NU = kLong ? (H + kDecThreads - 1) / kDecThreads : 1;
    float b0[NU][4], c0c[NU], c0n[NU];
    int r0[NU][4];
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const int ui = min(tid + kDecThreads * i, H - 1);
        c0c[i] = c0n[i] = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            b0[i][g] = p.b_ih[0][g * H + ui] + p.b_hh[0][g * H + ui];
            r0[i][g] = 0;
        }
    }

    int frame = 0, symbols = 0, last = blank, count = 0, steps = 0, alt = 0;
    bool emitted = false, valid = false;
    float pv[2 * KP];
    // long form: integer recurrent sums [layer][gate] of the committed state
    // (rs) and of the candidate (rs_next); the owning wave's cell states
    int rs[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}}, rs_next[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
    float c_cur[2] = {0.0f, 0.0f}, c_new[2] = {0.0f, 0.0f};
    while (frame < p.frames && !failed) {
        if (!valid) {
            pf_base = frame;  // the next round's window loads during this update's first barrier
            do_pf = true;
            if constexpr (!kLong) {
                // ---- two LSTM layers on the last token's embedding (zeros before any)
#pragma unroll
                for (int l = 0; l < 2; ++l) {
                    if (owns_unit) {
                        float x[2 * KP], hv[2 * KP];
#pragma unroll
                        for (int j = 0; j < KP; ++j) {
                            const int k = 2 * lane + 128 * j;
                            if (l == 0) {
                                if (emitted) {
                                    const uint32_t e = *(const uint32_t*)(p.emb + (size_t)last * H + k);
                                    x[2 * j] = lo16(e);
                                    x[2 * j + 1] = hi16(e);
                                } else {
                                    x[2 * j] = x[2 * j + 1] = 0.0f;
                                }
                            } else {
                                const float2 v = ld2(hp(alt ^ 1, 0) + k);  // this update's layer-0 output
                                x[2 * j] = v.x;
                                x[2 * j + 1] = v.y;
                            }
                            const float2 hh = ld2(hp(alt, l) + k);
                            hv[2 * j] = hh.x;
                            hv[2 * j + 1] = hh.y;
                        }
                        float s[4];
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            float a = 0.0f;
#pragma unroll
                            for (int j = 0; j < KP; ++j) {
                                a = __builtin_fmaf(lo16(wih[l][g][j]), x[2 * j], a);
                                a = __builtin_fmaf(hi16(wih[l][g][j]), x[2 * j + 1], a);
                                a = __builtin_fmaf(lo16(whh[l][g][j]), hv[2 * j], a);
                                a = __builtin_fmaf(hi16(whh[l][g][j]), hv[2 * j + 1], a);
                            }
                            s[g] = wave_sum(a) + bias[l][g];
                        }
                        if (lane == 0) {
                            const float ig = sigmoid(s[0]), fg = sigmoid(s[1]), cg = tanhf(s[2]), og = sigmoid(s[3]);
                            const float cell = fg * ld1(cp(alt, l) + u) + ig * cg;
                            st1(cp(alt ^ 1, l) + u, cell);
                            st1(hp(alt ^ 1, l) + u, og * tanhf(cell));
                        }
                    }
                    barrier(0);
                    if (failed) break;
                }
                if (failed) break;
                // ---- projection of the new layer-1 output
                if (owns_unit) {
                    float a = 0.0f;
#pragma unroll
                    for (int j = 0; j < KP; ++j) {
                        const float2 v = ld2(hp(alt ^ 1, 1) + 2 * lane + 128 * j);
                        a = __builtin_fmaf(lo16(wpj[j]), v.x, a);
                        a = __builtin_fmaf(hi16(wpj[j]), v.y, a);
                    }
                    a = wave_sum(a) + bpj;
                    if (lane == 0) st1(pred + u, a);
                }
            } else {
                // ---- layer 0 of every unit, in every workgroup: recurrent sums of the
                // committed state + bias + the token's table row (decoder.cu:619-648)
#pragma unroll
                for (int i = 0; i < NU; ++i) {
                    const int ui = tid + kDecThreads * i;
                    if (ui < H) {
                        float s[4];
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const float tv = emitted ? h2f(p.table[(size_t)last * 4 * H + g * H + ui]) : 0.0f;
                            s[g] = __builtin_fmaf((float)r0[i][g], cq[0], b0[i][g]) + tv;
                        }
                        float h;
                        lstm_cell(s, c0c[i], c0n[i], h);
                        ((uint8_t*)q0_s)[ui] = (uint8_t)quant_i8(h * 127.0f);
                    }
                }
                __syncthreads();
                // ---- layer 1: its recurrent sums + W_ih1 x the new INT8 layer-0
                // output (decoder.cu:650-670); the layer-0 recurrent sums of the new
                // candidate state go out for the update after it is committed
                if (owns_unit) {
                    uint32_t x[KD];
#pragma unroll
                    for (int j = 0; j < KD; ++j) x[j] = 4 * lane + 256 * j < H ? q0_s[lane + 64 * j] : 0u;
                    int in[4], r0n[4];
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        int a = 0, d = 0;
#pragma unroll
                        for (int j = 0; j < KD; ++j) {
                            a = __builtin_amdgcn_sdot4((int)qw[2][g][j], (int)x[j], a, false);
                            d = __builtin_amdgcn_sdot4((int)qw[0][g][j], (int)x[j], d, false);
                        }
                        in[g] = a;
                        r0n[g] = d;
                    }
#pragma unroll
                    for (int off = 1; off < 64; off <<= 1)
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            in[g] = add_level(in[g], off);
                            r0n[g] = add_level(r0n[g], off);
                        }
                    if (lane < 4) st_word((uint32_t*)rs0w + ((alt ^ 1) * H + u) * 4 + lane, (uint32_t)r0n[lane]);
                    if (lane == 0) {
                        float s[4];
#pragma unroll
                        for (int g = 0; g < 4; ++g)
                            s[g] = __builtin_fmaf((float)in[g], cq[2], __builtin_fmaf((float)rs[1][g], cq[1], bias[1][g]));
                        float h;
                        lstm_cell(s, c_cur[1], c_new[1], h);
                        st1(h1c + u, h);
                        qb_s[wave] = (uint32_t)(uint8_t)quant_i8(h * 127.0f);
                    }
                }
                __syncthreads();
                if (tid == 0 && 4 * blk < H)
                    st_word(qbank(alt ^ 1, 1) + blk, qb_s[0] | (qb_s[1] << 8) | (qb_s[2] << 16) | (qb_s[3] << 24));
                barrier(0);
                if (failed) break;
                // ---- projection of the new layer-1 output, and the layer-1 recurrent
                // sums of this candidate state for the update after it is committed
                if (owns_unit) {
                    uint32_t xq[KD];
#pragma unroll
                    for (int j = 0; j < KD; ++j) xq[j] = 4 * lane + 256 * j < H ? ld_word(qbank(alt ^ 1, 1) + lane + 64 * j) : 0u;
                    float a = 0.0f;
#pragma unroll
                    for (int j = 0; j < KP; ++j) {
                        const float2 v = ld2(h1c + 2 * lane + 128 * j);
                        a = __builtin_fmaf(lo16(wpj[j]), v.x, a);
                        a = __builtin_fmaf(hi16(wpj[j]), v.y, a);
                    }
                    a = wave_sum(a) + bpj;
                    if (lane == 0) st1(pred + u, a);
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        int d = 0;
#pragma unroll
                        for (int j = 0; j < KD; ++j) d = __builtin_amdgcn_sdot4((int)qw[1][g][j], (int)xq[j], d, false);
                        rs_next[1][g] = wave_isum(d);
                    }
                }
                // the candidate's layer-0 sums (published before the last barrier),
                // consumed by the next update once a token commits this state
#pragma unroll
                for (int i = 0; i < NU; ++i) {
                    const int ui = tid + kDecThreads * i;
                    if (ui < H)
#pragma unroll
                        for (int g = 0; g < 4; ++g) r0[i][g] = (int)ld_word((const uint32_t*)rs0w + ((alt ^ 1) * H + ui) * 4 + g);
                }
            }
            barrier(0);
            if (failed) break;
#pragma unroll
            for (int j = 0; j < KP; ++j) {
                const float2 v = ld2(pred + 2 * lane + 128 * j);
                pv[2 * j] = v.x;
                pv[2 * j + 1] = v.y;
            }
            valid = true;
        }
        // ---- joint round: frames frame .. frame + kWin - 1 against this prediction
        if (pf_base != frame) {
            pf_base = frame;
            prefetch();
        }
        {
            // the 2 x kWin dot products first, then their wave sums level by
            // level, so every butterfly step issues 2 kWin independent shuffles
            float acc[kWin][2];
#pragma unroll
            for (int c = 0; c < kWin; ++c) {
                float x[2 * KP];
#pragma unroll
                for (int j = 0; j < KP; ++j) {
                    const uint32_t ev = cand[c][j];
                    x[2 * j] = __builtin_fmaxf(lo16(ev) + pv[2 * j], 0.0f);
                    x[2 * j + 1] = __builtin_fmaxf(hi16(ev) + pv[2 * j + 1], 0.0f);
                }
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    float a = 0.0f;
#pragma unroll
                    for (int j = 0; j < KP; ++j) {
                        float w0, w1;
                        if constexpr (kInt8) {
                            w0 = (float)(int8_t)(wj[r][j] & 0xffu);
                            w1 = (float)(int8_t)((wj[r][j] >> 8) & 0xffu);
                        } else {
                            w0 = lo16(wj[r][j]);
                            w1 = hi16(wj[r][j]);
                        }
                        a = __builtin_fmaf(w0, x[2 * j], a);
                        a = __builtin_fmaf(w1, x[2 * j + 1], a);
                    }
                    acc[c][r] = a;
                }
            }
#pragma unroll
            for (int off = 1; off < 64; off <<= 1)
#pragma unroll
                for (int c = 0; c < kWin; ++c)
#pragma unroll
                    for (int r = 0; r < 2; ++r) acc[c][r] = add_level(acc[c][r], off);
#pragma unroll
            for (int c = 0; c < kWin; ++c) {
                float bs = -__builtin_huge_valf();
                int bi = 0x7fffffff;
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const float score = __builtin_fmaf(wjs[r], acc[c][r], wjb[r]);
                    const int id = jid[r];
                    if (id >= T) {
                        if (lane == 0) dur_sc[c][id - T] = score;  // workgroup 0 only
                    } else if (id >= 0) {
                        if (score > bs || (score == bs && id < bi)) {
                            bs = score;
                            bi = id;
                        }
                    }
                }
                if (lane == 0)
                    win_w[wave][c] = bi == 0x7fffffff ? 0ull
                                                      : (((unsigned long long)key_bits(bs) << 32) |
                                                         ((unsigned long long)(0xffffu - (uint32_t)bi) << 16));
            }
        }
        __syncthreads();
        // thread c: this workgroup's key for window frame c (workgroup 0's with
        // the first maximum of that frame's duration scores)
        unsigned long long key = 0ull;
        if (tid < kWin) {
            key = win_w[0][tid];
            for (int i = 1; i < 4; ++i) key = win_w[i][tid] > key ? win_w[i][tid] : key;
            if (blk == 0) {
                int d = 0;
                for (int i = 1; i < D; ++i)
                    if (dur_sc[tid][i] > dur_sc[tid][d]) d = i;
                key |= (unsigned long long)d << 13;
            }
        }
        // a blank run that leaves the window usually lands on its next frame:
        // that window loads during the barrier (a token's update reloads)
        pf_base = frame + kWin;
        do_pf = true;
        unsigned long long mine[kWin];
        barrier_win(key, mine);
        if (failed) break;
        // decisions of the window: per frame the largest key over the
        // workgroups is the best token; workgroup 0's carries the duration
        {
            if (tid == 0)
#pragma unroll
                for (int c = 0; c < kWin; ++c) win_dur[c] = (int)(((uint32_t)mine[c] >> 13) & 7u);
#pragma unroll
            for (int off = 1; off < 64; off <<= 1)
#pragma unroll
                for (int c = 0; c < kWin; ++c) {
                    mine[c] = max_level(mine[c], off);
                }
            if (lane == 0)
#pragma unroll
                for (int c = 0; c < kWin; ++c) win_w[wave][c] = mine[c];
            __syncthreads();
            if (tid < kWin) {
                unsigned long long b = win_w[0][tid];
                for (int i = 1; i < 4; ++i) b = win_w[i][tid] > b ? win_w[i][tid] : b;
                win_tok[tid] = (int)(0xffffu - (((uint32_t)b) >> 16));
            }
            __syncthreads();
            // the greedy rules (decoder.cu:773-783) over the window, identical in
            // every thread: blank decisions keep the prediction, so later frames'
            // decisions in the window stand until a token or the window's end
            const int f0 = frame;
            int c = 0;
            while (true) {
                const int token = win_tok[c], dur = win_dur[c];
                ++steps;
                if (token != blank) {
                    if (blk == 0 && tid == 0 && count < p.capacity) p.tokens[count] = token;
                    ++count;
                    last = token;
                    emitted = true;
                    valid = false;
                    alt ^= 1;  // the candidate state becomes the committed one
                    if constexpr (kLong) {
                        c_cur[1] = c_new[1];
#pragma unroll
                        for (int g = 0; g < 4; ++g) rs[1][g] = rs_next[1][g];
#pragma unroll
                        for (int i = 0; i < NU; ++i) c0c[i] = c0n[i];
                    }
                }
                ++symbols;
                frame += dur;
                if (dur != 0 || symbols == p.max_symbols) {
                    if (dur == 0) ++frame;
                    symbols = 0;
                }
                if (token != blank || frame >= p.frames) break;
                c = frame - f0;
                if (c >= kWin) break;
            }
            __syncthreads();  // win_w / win_tok / win_dur are reused next round
        }
    }
    if (blk == 0 && tid == 0) {
        p.result[0] = count;
        p.result[1] = frame;
        p.result[2] = failed ? -2 : 0;
        p.result[3] = steps;
    }
}

__global__ void decode_clear_kernel(uint32_t* ws, int words) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x) ws[i] = 0u;
}

}  // namespace

// fp16 form: h, c (2 banks x 2 layers) and the prediction; long form: INT8
// banks (H words), candidate layer-1 output (H), maxima (3 x blocks, <= 6H
// for H >= 128) and the prediction at the same offset 8H; after the joint
// rounds' words, the long form's layer-0 recurrent sums (2 banks x H x 4).
int decode_workspace_words(int hidden) { return kDecState + 9 * hidden + kDecExtWords + 8 * hidden; }

int launch_tdt_decode(const uint16_t* enc, int frames, int enc_stride, const uint16_t* emb, const uint16_t* table, const uint16_t* const* w_ih,
                      const uint16_t* const* w_hh, const float* const* b_ih, const float* const* b_hh, const uint16_t* w_proj,
                      const float* b_proj, const void* w_joint, int joint_int8, const float* joint_scales, const float* b_joint,
                      int hidden, int token_outputs, int durations, int max_symbols, int32_t* tokens, int capacity, int32_t* result,
                      uint32_t* workspace, hipStream_t s) {
    int blocks = cu_count();
    if (blocks > kDecMaxBlocks) blocks = kDecMaxBlocks;
    const int outputs = token_outputs + durations;
    if (hidden > 4 * blocks || outputs > 8 * blocks) {
        set_error("decode needs hidden <= %d and outputs <= %d on this GPU", 4 * blocks, 8 * blocks);
        return -1;
    }
    // only as many workgroups as own a hidden unit (4 each) or joint rows (8
    // each): every further one would only add a participant to each barrier
    const int needed = max((hidden + 3) / 4, (outputs + 7) / 8);
    if (needed < blocks) blocks = needed;
    if (hidden > 4 * blocks || outputs > 8 * blocks) {
        set_error("decode needs hidden <= %d and outputs <= %d on this GPU", 4 * blocks, 8 * blocks);
        return -1;
    }
    DecodeArgs a{};
    a.enc = enc;
    a.emb = emb;
    a.table = table;
    for (int l = 0; l < 2; ++l) {
        a.w_ih[l] = w_ih[l];
        a.w_hh[l] = w_hh[l];
        a.b_ih[l] = b_ih[l];
        a.b_hh[l] = b_hh[l];
    }
    a.w_proj = w_proj;
    a.b_proj = b_proj;
    a.w_joint = w_joint;
    a.joint_scales = joint_scales;
    a.b_joint = b_joint;
    a.tokens = tokens;
    a.result = result;
    a.ws = workspace;
    a.frames = frames;
    a.enc_stride = enc_stride;
    a.outputs = outputs;
    a.token_outputs = token_outputs;
    a.durations = durations;
    a.max_symbols = max_symbols;
    a.capacity = capacity;
    decode_clear_kernel<<<16, 256, 0, s>>>(workspace, decode_workspace_words(hidden));
    switch (hidden >> 7) {
#define PK_DEC_CASE(KP)                                                                          \
    case KP:                                                                                     \
        if (table) {                                                                             \
            if (joint_int8) tdt_decode_kernel<true, KP, true><<<blocks, kDecThreads, 0, s>>>(a);  \
            else tdt_decode_kernel<false, KP, true><<<blocks, kDecThreads, 0, s>>>(a);            \
        } else {                                                                                 \
            if (joint_int8) tdt_decode_kernel<true, KP, false><<<blocks, kDecThreads, 0, s>>>(a); \
            else tdt_decode_kernel<false, KP, false><<<blocks, kDecThreads, 0, s>>>(a);           \
        }                                                                                        \
        break;
        PK_DEC_CASE(1) PK_DEC_CASE(2) PK_DEC_CASE(3) PK_DEC_CASE(4) PK_DEC_CASE(5) PK_DEC_CASE(6) PK_DEC_CASE(7) PK_DEC_CASE(8)
#undef PK_DEC_CASE
    default: break;
    }
    return 0;
}

}  // namespace pk
