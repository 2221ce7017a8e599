// Long-form local relative-position attention of the Conformer encoder and
// the producers of its packed operands (encoder.cu:561-634, :1476-2097).
//
// Model constants (encoder.cu:12-17): width 1024 = 8 heads x 128, window
// 128 left / 128 right (257 keys), position table padded to 272 rows.
//
// A workgroup (256 threads, four waves) owns one 16-query tile of one head.
// Tiles whose whole key window lies inside [0, valid_rows) run the tile path:
// every 16 queries share the 272-key union qb-128 .. qb+143, so the scores
// are two 16x272 MFMA products (content q+u against the keys, position q+v
// against the 272 position rows) and the context is one 16x272x128 product.
//   packed: q+u -> INT4, keys INT4, q+v -> INT8, positions INT8, all on
//           v_mfma_i32_16x16x64_i8 (signed nibbles are widened to the high
//           half of a byte, i.e. times 16, and the exact sums shifted back);
//           U4 probabilities x S4 values on the same instruction.
//   tc:     fp16 scores on v_mfma_f32_16x16x32_f16; e4m3 probabilities x
//           e4m3 values on v_mfma_scale_f32_16x16x128_f8f6f4.
// Boundary tiles run the per-query FP32 path: one 32-lane half wave per
// query, with the score, maximum and denominator reductions in the order of
// the reference's 32-lane warps.
//
// The MFMA reduction dimension may be permuted freely as long as both
// operands use the same permutation (integer sums are exact).  The key and
// position vectors keep the byte order of the reference packers so that the
// packed buffers are interchangeable; the queries are quantized inside the
// kernel directly into the matching operand order.
#include <float.h>

#include "pk_common.hpp"
#include "pk_kernels.hpp"

namespace pk {
namespace {

constexpr int kModel = 1024, kHead = 128, kHeads = 8;
constexpr int kMaxAtt = 257, kPosRows = 272;
constexpr float kScoreScale = 0.08838834764831845f;  // 1/sqrt(128)
constexpr float kValueScale = 8.0f / 448.0f;         // FP8 V holds v * 56

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint16_t bf16_rn(float v) {  // finite inputs only
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf16_f32(uint16_t h) { return __builtin_bit_cast(float, (uint32_t)h << 16); }

// Eight signed nibbles -> two words of four bytes, each nibble in the high
// half of its byte (value * 16): lo takes the even nibbles, hi the odd ones.
__device__ __forceinline__ uint32_t nib_lo16(uint32_t w) { return (w << 4) & 0xf0f0f0f0u; }
__device__ __forceinline__ uint32_t nib_hi16(uint32_t w) { return w & 0xf0f0f0f0u; }
__device__ __forceinline__ v4i widen_s4x16(uint2 w) {
    return v4i{(int)nib_lo16(w.x), (int)nib_hi16(w.x), (int)nib_lo16(w.y), (int)nib_hi16(w.y)};
}

// Position of key k (0..319, relative to the tile's first key) in a row of
// the U4 probability operand: within each 16 keys the order is
// 0,2,4,6, 1,3,5,7, 8,10,12,14, 9,11,13,15, which is the order widen_s4x16
// produces from 16 consecutive S4 values.
__device__ __forceinline__ int prob_pos(int k) { return (k & ~15) + (k & 8) + ((k & 1) << 2) + ((k & 7) >> 1); }

// ---- packers ------------------------------------------------------------

// encoder.cu:2054-2074 / :2076-2097.  16 lanes per 128-value vector, lane j
// holding dimensions 8j..8j+7.  INT8: dims 8j..8j+3 go to the four bytes of
// reference lane 2j, 8j+4..8j+7 to those of lane 2j+1.  INT4: both reference
// lanes' u16 words are adjacent, so the eight nibbles form one u32 at
// (j/8)*32 + (j%4)*8 + (j&4).
template <bool kInt4>
__global__ __launch_bounds__(256) void pack_vectors_kernel(const uint16_t* __restrict__ in, uint8_t* __restrict__ out,
                                                           float* __restrict__ scales, int vectors) {
    const int vec = (int)(blockIdx.x * 16 + (threadIdx.x >> 4));
    const int j = threadIdx.x & 15;
    if (vec >= vectors) return;
    const uint4 raw = *(const uint4*)(in + (size_t)vec * 128 + 8 * j);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    float v[8], m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[i] = h2f((uint16_t)(w[i / 2] >> (16 * (i & 1))));
        m = __builtin_fmaxf(m, __builtin_fabsf(v[i]));
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) m = __builtin_fmaxf(m, __shfl_xor(m, off, 64));
    const float scale = m > 0.0f ? m / (kInt4 ? 7.0f : 127.0f) : 1.0f;
    if (j == 0) scales[vec] = scale;
    if constexpr (kInt4) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) word |= ((uint32_t)(int)__builtin_rintf(v[i] / scale) & 15u) << (4 * i);
        *(uint32_t*)(out + (size_t)vec * 64 + (j / 8) * 32 + (j % 4) * 8 + (j & 4)) = word;
    } else {
        uint32_t word[2] = {0, 0};
#pragma unroll
        for (int i = 0; i < 8; ++i) word[i / 4] |= ((uint32_t)(int)__builtin_rintf(v[i] / scale) & 255u) << (8 * (i & 3));
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int lane = 2 * j + h;
            *(uint32_t*)(out + (size_t)vec * 128 + (lane / 8) * 32 + (lane % 4) * 8 + (lane & 4)) = word[h];
        }
    }
}

// encoder.cu:561-634.  One 1024-thread workgroup per feature row of the
// feature-major V [1024 x rows]; each thread handles 8 consecutive keys per
// chunk.  With kResident the row stays in registers between the maximum and
// the quantization pass (rows <= 49152); otherwise it is read twice.
constexpr int kValueChunks = 6;
template <bool kResident>
__global__ __launch_bounds__(1024) void quantize_value_int4_kernel(const uint16_t* __restrict__ vt, uint8_t* __restrict__ out,
                                                                   int rows, float inverse_scale, int edge_only,
                                                                   int valid_rows) {
    const int f = blockIdx.x, tid = threadIdx.x;
    const size_t elements = (size_t)rows * kModel;
    const uint16_t* x = vt + (size_t)f * rows;
    __shared__ float wave_max_s[16];
    __shared__ float scale_s;
    uint4 held[kResident ? kValueChunks : 1];
    float m = 0.0f;
    const int chunks = (rows + 8191) / 8192;
    for (int c = 0; c < (kResident ? kValueChunks : chunks); ++c) {
        const int r = c * 8192 + 8 * tid;
        uint4 u = uint4{0, 0, 0, 0};
        if (r < rows) u = *(const uint4*)(x + r);
        if constexpr (kResident) held[c] = u;
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) m = __builtin_fmaxf(m, __builtin_fabsf(h2f((uint16_t)(w[i / 2] >> (16 * (i & 1))))));
    }
    m = wave_max(m);
    if ((tid & 63) == 0) wave_max_s[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) {
        float t = 0.0f;
        for (int i = 0; i < 16; ++i) t = __builtin_fmaxf(t, wave_max_s[i]);
        const float s = t > 0.0f ? t / 7.0f : 1.0f;
        scale_s = s;
        ((float*)(out + elements + elements / 2))[f] = s;
    }
    __syncthreads();
    const float scale = scale_s;
    for (int c = 0; c < (kResident ? kValueChunks : chunks); ++c) {
        const int r = c * 8192 + 8 * tid;
        if (r >= rows) break;
        uint4 u;
        if constexpr (kResident) u = held[c];
        else u = *(const uint4*)(x + r);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
        uint32_t fp8[2] = {0, 0}, s4 = 0;
        bool all = true;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const float a = h2f((uint16_t)(w[p] & 0xffffu)), b = h2f((uint16_t)(w[p] >> 16));
            fp8[p / 2] |= e4m3x2(a * inverse_scale, b * inverse_scale) << (16 * (p & 1));
            const int qa = rne_clamp(a / scale, -7, 7), qb = rne_clamp(b / scale, -7, 7);
            s4 |= (uint32_t)((qa & 15) | ((qb & 15) << 4)) << (8 * p);
            const int row = r + 2 * p;
            all = all && (!edge_only || row < 272 || row + 1 >= valid_rows - 272);
        }
        *(uint32_t*)(out + elements + ((size_t)f * rows + r) / 2) = s4;
        uint8_t* o = out + (size_t)f * rows + r;
        if (all) {
            *(uint2*)o = uint2{fp8[0], fp8[1]};
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int row = r + 2 * p;
                if (row < 272 || row + 1 >= valid_rows - 272) *(uint16_t*)(o + 2 * p) = (uint16_t)(fp8[p / 2] >> (16 * (p & 1)));
            }
        }
    }
}

// ---- attention -----------------------------------------------------------

struct ScalarShared {
    float scores[8][264];
};
struct PackedShared {
    uint8_t qa_u[16][144];  // INT4 (q+u) as int8, MFMA operand order, rows padded
    uint8_t qa_v[16][144];  // INT8 (q+v), reference score-vector byte order
    uint16_t cs[16][kPosRows];
    uint16_t ps[16][kPosRows];
    uint8_t prob[16][336];  // U4 probabilities as bytes, prob_pos order
    uint8_t out[16][128];
    float qs_u[16], qs_v[16], pscale[16];
};
struct TcShared {
    uint16_t qu[16][136];
    uint16_t qv[16][136];
    float cs[16][kPosRows];
    float ps[16][kPosRows];
    uint8_t prob[16][400];  // e4m3 probabilities for keys 0..383 (zero past the window)
    uint16_t out[16][128];
};
// Each kernel instantiation declares only the union it uses, so the packed
// kernel's LDS (and occupancy) does not pay for the fp32 score planes.
union PackedAttnShared {
    ScalarShared s;
    PackedShared p;
};
union TcAttnShared {
    ScalarShared s;
    TcShared t;
};

// Context store (encoder.cu:1463-1474): fp16 round, packed form e4m3(x * 28).
template <bool kPacked>
__device__ __forceinline__ void store4(void* output, size_t index, const float (&c)[4]) {
    if constexpr (kPacked) {
        const uint32_t lo = e4m3x2(round_f16(c[0]) * 28.0f, round_f16(c[1]) * 28.0f);
        const uint32_t hi = e4m3x2(round_f16(c[2]) * 28.0f, round_f16(c[3]) * 28.0f);
        *(uint32_t*)((uint8_t*)output + index) = lo | (hi << 16);
    } else {
        const uint32_t lo = (uint32_t)f2h(c[0]) | ((uint32_t)f2h(c[1]) << 16);
        const uint32_t hi = (uint32_t)f2h(c[2]) | ((uint32_t)f2h(c[3]) << 16);
        *(uint2*)((uint16_t*)output + index) = uint2{lo, hi};
    }
}

// encoder.cu:1548-1684: per-query FP32 path, one half wave per query.
template <bool kPacked>
__device__ void attention_scalar(ScalarShared& sh, const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
                                 const uint8_t* __restrict__ value_fp8, const uint16_t* __restrict__ position,
                                 const uint16_t* __restrict__ bias_u, const uint16_t* __restrict__ bias_v, void* output,
                                 int qb, int head, int rows, int padded_rows, int valid_rows, int left, int right,
                                 int value_stride) {
    const int hw = threadIdx.x >> 5, ln = threadIdx.x & 31;
    float* scores = sh.scores[hw];
    for (int lq = hw; lq < 16; lq += 8) {
        const int qr = qb + lq;
        const size_t oidx = (size_t)qr * kModel + head * kHead + 4 * ln;
        if (qr >= rows || qr >= valid_rows) {
            if (qr < padded_rows) {
                const float z[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                store4<kPacked>(output, oidx, z);
            }
            continue;
        }
        const int first = max(0, qr - left), last = min(valid_rows - 1, qr + right);
        const int count = last - first + 1;
        const int half = ln >> 4, hl = ln & 15;
        float2 su[4], sv[4];
#pragma unroll
        for (int quarter = 0; quarter < 4; ++quarter) {
            const int d = head * kHead + 2 * hl + 32 * quarter;
            const uint32_t q = *(const uint32_t*)(query + (size_t)qr * kModel + d);
            const uint32_t u = *(const uint32_t*)(bias_u + d);
            const uint32_t v = *(const uint32_t*)(bias_v + d);
            const float q0 = h2f((uint16_t)q), q1 = h2f((uint16_t)(q >> 16));
            su[quarter] = make_float2(q0 + h2f((uint16_t)u), q1 + h2f((uint16_t)(u >> 16)));
            sv[quarter] = make_float2(q0 + h2f((uint16_t)v), q1 + h2f((uint16_t)(v >> 16)));
        }
        for (int sp = 0; sp < count; sp += 2) {
            const int slot = sp + half;
            const int key_row = first + min(slot, count - 1);
            const int prow = left - qr + key_row;
            float s = 0.0f;
#pragma unroll
            for (int quarter = 0; quarter < 4; ++quarter) {
                const int d = 2 * hl + 32 * quarter;
                const uint32_t k = *(const uint32_t*)(key + (size_t)key_row * kModel + head * kHead + d);
                const uint32_t p = *(const uint32_t*)(position + ((size_t)head * kPosRows + prow) * kHead + d);
                s = __builtin_fmaf(su[quarter].x, h2f((uint16_t)k), s);
                s = __builtin_fmaf(sv[quarter].x, h2f((uint16_t)p), s);
                s = __builtin_fmaf(su[quarter].y, h2f((uint16_t)(k >> 16)), s);
                s = __builtin_fmaf(sv[quarter].y, h2f((uint16_t)(p >> 16)), s);
            }
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
            if (hl == 0 && slot < count) scores[slot] = s * kScoreScale;
        }
        wave_sync();
        float mx = -FLT_MAX;
        for (int slot = ln; slot < count; slot += 32) mx = __builtin_fmaxf(mx, scores[slot]);
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, off, 64));
        float den = 0.0f;
        for (int slot = ln; slot < count; slot += 32) {
            const float e = expf(scores[slot] - mx);
            scores[slot] = e;
            den += e;
        }
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) den += __shfl_xor(den, off, 64);
        den = __shfl(den, 0, 32);
        wave_sync();
        float c[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const int feature = head * kHead + 4 * ln;
        for (int chunk = first & ~3; chunk <= last; chunk += 4) {
            uint32_t words[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) words[i] = *(const uint32_t*)(value_fp8 + (size_t)(feature + i) * value_stride + chunk);
#pragma unroll
            for (int item = 0; item < 4; ++item) {
                const int kr = chunk + item;
                if (kr < first || kr > last) continue;
                const float weight = scores[kr - first] / den;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    c[i] = __builtin_fmaf(weight, e4m3_to_f32((words[i] >> (8 * item)) & 0xffu) * kValueScale, c[i]);
            }
        }
        store4<kPacked>(output, oidx, c);
        wave_sync();
    }
}

// Softmax of query lq over its 257 slots from the combined logits held by a
// half wave (lane ln has slots ln + 32 part).  Returns e = exp(l - max) in
// place and the denominator (shuffle tree in 32-lane warp order).
__device__ __forceinline__ float softmax_half(float (&l)[9], int ln) {
    float mx = -FLT_MAX;
#pragma unroll
    for (int part = 0; part < 9; ++part)
        if (ln + 32 * part < kMaxAtt) mx = __builtin_fmaxf(mx, l[part]);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, off, 64));
    float den = 0.0f;
#pragma unroll
    for (int part = 0; part < 9; ++part)
        if (ln + 32 * part < kMaxAtt) {
            l[part] = expf(l[part] - mx);
            den += l[part];
        }
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) den += __shfl_xor(den, off, 64);
    return __shfl(den, 0, 32);
}

// encoder.cu:1687-1966: INT4/INT8 scores, U4 x S4 context, e4m3(x*28) out.
__device__ void attention_packed_tile(PackedShared& sh, const uint16_t* __restrict__ query, const uint8_t* __restrict__ value_fp8,
                                      const uint16_t* __restrict__ bias_u, const uint16_t* __restrict__ bias_v,
                                      uint8_t* __restrict__ output, int qb, int head, int value_stride,
                                      const uint8_t* __restrict__ packed_key, const float* __restrict__ key_scales,
                                      const uint8_t* __restrict__ packed_position, const float* __restrict__ position_scales) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, l16 = lane & 15;
    const int first_key = qb - 128;

    // Phase 1: clear the probability rows; quantize q+u and q+v.
    for (int i = tid; i < 16 * 336 / 4; i += 256) ((uint32_t*)sh.prob)[i] = 0;
    {
        const int r = tid >> 4, j = tid & 15;
        const size_t qi = (size_t)(qb + r) * kModel + head * kHead + 8 * j;
        const uint4 q = *(const uint4*)(query + qi);
        const uint4 u = *(const uint4*)(bias_u + head * kHead + 8 * j);
        const uint4 v = *(const uint4*)(bias_v + head * kHead + 8 * j);
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w}, uw[4] = {u.x, u.y, u.z, u.w}, vw[4] = {v.x, v.y, v.z, v.w};
        float vu[8], vv[8], mu = 0.0f, mv = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int sh16 = 16 * (i & 1);
            const float qf = h2f((uint16_t)(qw[i / 2] >> sh16));
            vu[i] = round_f16(qf + h2f((uint16_t)(uw[i / 2] >> sh16)));
            vv[i] = round_f16(qf + h2f((uint16_t)(vw[i / 2] >> sh16)));
            mu = __builtin_fmaxf(mu, __builtin_fabsf(vu[i]));
            mv = __builtin_fmaxf(mv, __builtin_fabsf(vv[i]));
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            mu = __builtin_fmaxf(mu, __shfl_xor(mu, off, 64));
            mv = __builtin_fmaxf(mv, __shfl_xor(mv, off, 64));
        }
        const float su = mu > 0.0f ? mu / 7.0f : 1.0f, sv = mv > 0.0f ? mv / 127.0f : 1.0f;
        if (j == 0) {
            sh.qs_u[r] = su;
            sh.qs_v[r] = sv;
        }
        uint32_t ue = 0, uo = 0, v8[2] = {0, 0};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t a = (uint32_t)(int)__builtin_rintf(vu[i] / su) & 255u;
            if (i & 1) uo |= a << (8 * (i >> 1));
            else ue |= a << (8 * (i >> 1));
            v8[i / 4] |= ((uint32_t)(int)__builtin_rintf(vv[i] / sv) & 255u) << (8 * (i & 3));
        }
        // INT4 plane: dimension 8j+i sits at storage nibble 2*off_j + i of the
        // key vectors; widen_s4x16 of the key's bytes [32m + 8g', +8) yields
        // even nibbles then odd nibbles per word, hence this operand order.
        const int pa = 64 * (j >> 3) + 16 * (j & 3) + 8 * ((j >> 2) & 1);
        *(uint2*)&sh.qa_u[r][pa] = uint2{ue, uo};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int L = 2 * j + h;
            *(uint32_t*)&sh.qa_v[r][(L / 8) * 32 + (L % 4) * 8 + (L & 4)] = v8[h];
        }
    }
    __syncthreads();

    // Phase 2: scores for the 17 key tiles of 16 columns, four waves.
    {
        const v4i au0 = __builtin_bit_cast(v4i, *(const uint4*)&sh.qa_u[l16][16 * g]);
        const v4i au1 = __builtin_bit_cast(v4i, *(const uint4*)&sh.qa_u[l16][64 + 16 * g]);
        const v4i av0 = __builtin_bit_cast(v4i, *(const uint4*)&sh.qa_v[l16][16 * g]);
        const v4i av1 = __builtin_bit_cast(v4i, *(const uint4*)&sh.qa_v[l16][64 + 16 * g]);
        float qsu[4], qsv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            qsu[r] = sh.qs_u[4 * g + r];
            qsv[r] = sh.qs_v[4 * g + r];
        }
        for (int kt = wave; kt < kPosRows / 16; kt += 4) {
            const int col = 16 * kt + l16;
            const int kvec = (first_key + col) * kHeads + head;
            const int pvec = head * kPosRows + col;
            const uint8_t* kb = packed_key + (size_t)kvec * 64;
            const uint8_t* pb = packed_position + (size_t)pvec * 128;
            const uint2 k0 = *(const uint2*)(kb + 8 * g), k1 = *(const uint2*)(kb + 32 + 8 * g);
            const uint4 p0 = *(const uint4*)(pb + 16 * g), p1 = *(const uint4*)(pb + 64 + 16 * g);
            const float ks = key_scales[kvec], pscl = position_scales[pvec];
            v4i acu = __builtin_amdgcn_mfma_i32_16x16x64_i8(au0, widen_s4x16(k0), v4i{0, 0, 0, 0}, 0, 0, 0);
            acu = __builtin_amdgcn_mfma_i32_16x16x64_i8(au1, widen_s4x16(k1), acu, 0, 0, 0);
            v4i acv = __builtin_amdgcn_mfma_i32_16x16x64_i8(av0, __builtin_bit_cast(v4i, p0), v4i{0, 0, 0, 0}, 0, 0, 0);
            acv = __builtin_amdgcn_mfma_i32_16x16x64_i8(av1, __builtin_bit_cast(v4i, p1), acv, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sh.cs[4 * g + r][col] = bf16_rn((float)(acu[r] >> 4) * (qsu[r] * ks));
                sh.ps[4 * g + r][col] = bf16_rn((float)acv[r] * (qsv[r] * pscl));
            }
        }
    }
    __syncthreads();

    // Phase 3: softmax and U4 probabilities, one half wave per query.
    {
        const int hw = tid >> 5, ln = tid & 31;
#pragma unroll
        for (int item = 0; item < 2; ++item) {
            const int lq = hw + 8 * item;
            float l[9];
#pragma unroll
            for (int part = 0; part < 9; ++part) {
                const int slot = ln + 32 * part;
                l[part] = slot < kMaxAtt ? (bf16_f32(sh.cs[lq][lq + slot]) + bf16_f32(sh.ps[lq][slot])) * kScoreScale : -FLT_MAX;
            }
            const float den = softmax_half(l, ln);
            if (ln == 0) sh.pscale[lq] = 1.0f / (15.0f * den);
#pragma unroll
            for (int part = 0; part < 9; ++part) {
                const int slot = ln + 32 * part;
                if (slot < kMaxAtt) sh.prob[lq][prob_pos(lq + slot)] = (uint8_t)(int)__builtin_rintf(l[part] * 15.0f);
            }
        }
    }
    __syncthreads();

    // Phase 4: context = U4 probabilities x S4 V over keys 0..271 (five K=64
    // steps; keys >= 272 contribute zero operands).
    {
        const uint8_t* s4 = value_fp8 + (size_t)kModel * value_stride;
        const float* vscales = (const float*)(value_fp8 + (size_t)kModel * value_stride * 3 / 2);
        v4i acc[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
#pragma unroll
        for (int s = 0; s < 5; ++s) {
            const int ko = 64 * s + 16 * g;
            const v4i a = __builtin_bit_cast(v4i, *(const uint4*)&sh.prob[l16][ko]);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int fg = head * kHead + 16 * (2 * wave + c) + l16;
                uint2 w = uint2{0, 0};
                if (ko < kPosRows) w = *(const uint2*)(s4 + ((size_t)fg * value_stride + first_key + ko) / 2);
                acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, widen_s4x16(w), acc[c], 0, 0, 0);
            }
        }
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int fl = 16 * (2 * wave + c) + l16;
            const float vs = vscales[head * kHead + fl];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 4 * g + r;
                const float x = (float)(acc[c][r] >> 4) * (sh.pscale[row] * vs);
                sh.out[row][fl] = (uint8_t)e4m3x2(round_f16(x) * 28.0f, 0.0f);
            }
        }
    }
    __syncthreads();
    {
        const int r = tid >> 4, j = tid & 15;
        *(uint2*)(output + (size_t)(qb + r) * kModel + head * kHead + 8 * j) = *(const uint2*)&sh.out[r][8 * j];
    }
}

// encoder.cu:1768-2018 (kPackedOutput = false): fp16 scores, e4m3 probabilities
// (p * 448) x e4m3 V, scaled by (1/448)*(8/448), fp16 out.
__device__ void attention_tc_tile(TcShared& sh, const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
                                  const uint8_t* __restrict__ value_fp8, const uint16_t* __restrict__ position,
                                  const uint16_t* __restrict__ bias_u, const uint16_t* __restrict__ bias_v,
                                  uint16_t* __restrict__ output, int qb, int head, int value_stride) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, l16 = lane & 15;
    const int first_key = qb - 128;
    {
        const int r = tid >> 4, j = tid & 15;
        const uint4 q = *(const uint4*)(query + (size_t)(qb + r) * kModel + head * kHead + 8 * j);
        const uint4 u = *(const uint4*)(bias_u + head * kHead + 8 * j);
        const uint4 v = *(const uint4*)(bias_v + head * kHead + 8 * j);
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w}, uw[4] = {u.x, u.y, u.z, u.w}, vw[4] = {v.x, v.y, v.z, v.w};
        uint32_t ou[4], ov[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float q0 = h2f((uint16_t)qw[i]), q1 = h2f((uint16_t)(qw[i] >> 16));
            ou[i] = (uint32_t)f2h(q0 + h2f((uint16_t)uw[i])) | ((uint32_t)f2h(q1 + h2f((uint16_t)(uw[i] >> 16))) << 16);
            ov[i] = (uint32_t)f2h(q0 + h2f((uint16_t)vw[i])) | ((uint32_t)f2h(q1 + h2f((uint16_t)(vw[i] >> 16))) << 16);
        }
        *(uint4*)&sh.qu[r][8 * j] = uint4{ou[0], ou[1], ou[2], ou[3]};
        *(uint4*)&sh.qv[r][8 * j] = uint4{ov[0], ov[1], ov[2], ov[3]};
    }
    __syncthreads();
    {
        v8h au[4], av[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            au[m] = __builtin_bit_cast(v8h, *(const uint4*)&sh.qu[l16][32 * m + 8 * g]);
            av[m] = __builtin_bit_cast(v8h, *(const uint4*)&sh.qv[l16][32 * m + 8 * g]);
        }
        for (int kt = wave; kt < kPosRows / 16; kt += 4) {
            const int col = 16 * kt + l16;
            const uint16_t* kr = key + (size_t)(first_key + col) * kModel + head * kHead + 8 * g;
            const uint16_t* pr = position + ((size_t)head * kPosRows + col) * kHead + 8 * g;
            uint4 kb[4], pb[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                kb[m] = *(const uint4*)(kr + 32 * m);
                pb[m] = *(const uint4*)(pr + 32 * m);
            }
            v4f acu = v4f{0, 0, 0, 0}, acv = v4f{0, 0, 0, 0};
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                acu = __builtin_amdgcn_mfma_f32_16x16x32_f16(au[m], __builtin_bit_cast(v8h, kb[m]), acu, 0, 0, 0);
                acv = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[m], __builtin_bit_cast(v8h, pb[m]), acv, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sh.cs[4 * g + r][col] = acu[r];
                sh.ps[4 * g + r][col] = acv[r];
            }
        }
    }
    __syncthreads();
    {
        const int hw = tid >> 5, ln = tid & 31;
#pragma unroll
        for (int item = 0; item < 2; ++item) {
            const int lq = hw + 8 * item;
            float l[9];
#pragma unroll
            for (int part = 0; part < 9; ++part) {
                const int slot = ln + 32 * part;
                l[part] = slot < kMaxAtt ? (sh.cs[lq][lq + slot] + sh.ps[lq][slot]) * kScoreScale : -FLT_MAX;
            }
            const float den = softmax_half(l, ln);
            // Union slot u = lq + slot; bytes outside the window are e4m3(0).
            for (int u = ln; u < 384; u += 32) sh.prob[lq][u] = 0;
            wave_sync();
#pragma unroll
            for (int part = 0; part < 9; ++part) {
                const int slot = ln + 32 * part;
                if (slot < kMaxAtt) sh.prob[lq][lq + slot] = (uint8_t)e4m3x2(l[part] / den * 448.0f, 0.0f);
            }
        }
    }
    __syncthreads();
    {
        v4f acc[2] = {v4f{0, 0, 0, 0}, v4f{0, 0, 0, 0}};
#pragma unroll
        for (int s = 0; s < 3; ++s) {
            const int ko = 128 * s + 32 * g;
            const uint4 a0 = *(const uint4*)&sh.prob[l16][ko], a1 = *(const uint4*)&sh.prob[l16][ko + 16];
            const v8i a = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int fg = head * kHead + 16 * (2 * wave + c) + l16;
                const uint8_t* vr = value_fp8 + (size_t)fg * value_stride + first_key + ko;
                uint4 b0 = uint4{0, 0, 0, 0}, b1 = uint4{0, 0, 0, 0};
                if (ko < kPosRows) b0 = *(const uint4*)vr;
                if (ko + 16 < kPosRows) b1 = *(const uint4*)(vr + 16);
                const v8i b = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
                acc[c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[c], 0, 0, 0, 0, 0, 0);
            }
        }
        constexpr float kContextScale = (1.0f / 448.0f) * (8.0f / 448.0f);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int fl = 16 * (2 * wave + c) + l16;
#pragma unroll
            for (int r = 0; r < 4; ++r) sh.out[4 * g + r][fl] = f2h(acc[c][r] * kContextScale);
        }
    }
    __syncthreads();
    {
        const int r = tid >> 4, j = tid & 15;
        *(uint4*)(output + (size_t)(qb + r) * kModel + head * kHead + 8 * j) = *(const uint4*)&sh.out[r][8 * j];
    }
}

template <bool kPacked>
__global__ __launch_bounds__(256) void local_attention_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ key, const uint8_t* __restrict__ value_fp8,
    const uint16_t* __restrict__ position, const uint16_t* __restrict__ bias_u, const uint16_t* __restrict__ bias_v,
    void* __restrict__ output, int rows, int padded_rows, int valid_rows, int left, int right, int value_stride,
    const uint8_t* __restrict__ packed_key, const float* __restrict__ key_scales, const uint8_t* __restrict__ packed_position,
    const float* __restrict__ position_scales) {
    const int qb = (int)blockIdx.x * 16, head = (int)blockIdx.y;
    if (qb >= padded_rows) return;
    const bool interior = qb >= left && qb + 15 + right < valid_rows && qb + 16 <= rows;
    if constexpr (kPacked) {
        __shared__ PackedAttnShared sh;
        if (!interior)
            attention_scalar<true>(sh.s, query, key, value_fp8, position, bias_u, bias_v, output, qb, head, rows, padded_rows,
                                   valid_rows, left, right, value_stride);
        else
            attention_packed_tile(sh.p, query, value_fp8, bias_u, bias_v, (uint8_t*)output, qb, head, value_stride, packed_key,
                                  key_scales, packed_position, position_scales);
    } else {
        __shared__ TcAttnShared sh;
        if (!interior)
            attention_scalar<false>(sh.s, query, key, value_fp8, position, bias_u, bias_v, output, qb, head, rows, padded_rows,
                                    valid_rows, left, right, value_stride);
        else
            attention_tc_tile(sh.t, query, key, value_fp8, position, bias_u, bias_v, (uint16_t*)output, qb, head, value_stride);
    }
}

}  // namespace

int launch_pack_vectors(bool int4, const uint16_t* in, uint8_t* out, float* scales, int vectors, hipStream_t s) {
    if (vectors <= 0) return 0;
    const dim3 grid((unsigned)((vectors + 15) / 16));
    if (int4) pack_vectors_kernel<true><<<grid, 256, 0, s>>>(in, out, scales, vectors);
    else pack_vectors_kernel<false><<<grid, 256, 0, s>>>(in, out, scales, vectors);
    return 0;
}

int launch_quantize_value_int4(const uint16_t* vt, uint8_t* out, int rows, float inverse_scale, bool edge_only, int valid_rows,
                               hipStream_t s) {
    if (rows <= kValueChunks * 8192)
        quantize_value_int4_kernel<true><<<kModel, 1024, 0, s>>>(vt, out, rows, inverse_scale, edge_only ? 1 : 0, valid_rows);
    else
        quantize_value_int4_kernel<false><<<kModel, 1024, 0, s>>>(vt, out, rows, inverse_scale, edge_only ? 1 : 0, valid_rows);
    return 0;
}

int launch_local_attention(bool packed, const uint16_t* query, const uint16_t* key, const uint8_t* value_fp8,
                           const uint16_t* position, const uint16_t* bias_u, const uint16_t* bias_v, void* output, int rows,
                           int padded_rows, int valid_rows, int left, int right, int value_stride, const uint8_t* packed_key,
                           const float* key_scales, const uint8_t* packed_position, const float* position_scales, hipStream_t s) {
    const dim3 grid((unsigned)((padded_rows + 15) / 16), kHeads);
    if (packed)
        local_attention_kernel<true><<<grid, 256, 0, s>>>(query, key, value_fp8, position, bias_u, bias_v, output, rows, padded_rows,
                                                          valid_rows, left, right, value_stride, packed_key, key_scales,
                                                          packed_position, position_scales);
    else
        local_attention_kernel<false><<<grid, 256, 0, s>>>(query, key, value_fp8, position, bias_u, bias_v, output, rows,
                                                           padded_rows, valid_rows, left, right, value_stride, nullptr, nullptr,
                                                           nullptr, nullptr);
    return 0;
}

}  // namespace pk
