// Short-form local relative-position attention (encoder.cu:1338-1461, the
// reference's kernel for padded_rows < 512, encoder.rs:619,850-858) and two
// layout kernels of the attention path: the fixed-scale e4m3 transpose of V
// for the tc attention (encoder.cu:644-671, encoder.rs:826-836) and the
// per-head position packer of the cached position projections
// (encoder.cu:1321-1336, encoder.rs:442-480).
//
// Short attention: one wave64 per (query, head).  Scores: the 64 lanes form
// four 16-lane groups, each lane holding 8 of the head's 128 dimensions as one
// 16-byte load of K and of the packed position row, so one pass scores four
// keys; a 16-lane DPP row sum gives each key's score, scaled by 1/sqrt(128)
// and kept in the wave's LDS row.  Softmax over the <= 257 scores with the
// wave's max and sum, then the context: lane l accumulates dimensions 2l and
// 2l+1 over the keys, probability = exp(s - max) / sum, as the reference.
#include "pk_kernels.hpp"

namespace pk {

namespace {

constexpr int kModel = 1024, kHeadW = 128, kHeadsN = 8, kPosRows = 272;
constexpr int kMaxKeys = 257;

// Sum over a DPP row of 16 lanes, valid in the row's lane 0 (row_shl n gives
// lane i the value of lane i + n of its row, 0 past the row's end).
template <int N>
__device__ __forceinline__ float row_shl(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + N, 0xf, 0xf, true));
}
__device__ __forceinline__ float row_sum16(float v) {
    v += row_shl<8>(v);
    v += row_shl<4>(v);
    v += row_shl<2>(v);
    return v + row_shl<1>(v);
}

__device__ __forceinline__ void wave_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// out[f * rows + r] = e4m3(in[r * 1024 + f] * inverse_scale), a 64 x 64 tile
// per workgroup through LDS so that both the fp16 reads (128 bytes of a row)
// and the byte writes (64 bytes of an output row) are contiguous.
__global__ __launch_bounds__(256) void quantize_fp8_transpose_kernel(const uint16_t* __restrict__ in, uint8_t* __restrict__ out,
                                                                     int rows, float inv) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[64][64 + 16];  // [feature][row]
    const int f0 = blockIdx.x * 64, r0 = blockIdx.y * 64, tid = threadIdx.x;
    {
        const int r = tid >> 2, c = (tid & 3) * 16, row = r0 + r;
        if (row < rows) {
            const uint4* src = (const uint4*)(in + (size_t)row * kModel + f0 + c);
            const uint4 a = src[0], b = src[1];
            const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t pair = e4m3x2(h2f((uint16_t)(w[i] & 0xffffu)) * inv, h2f((uint16_t)(w[i] >> 16)) * inv);
                tile[c + 2 * i][r] = (uint8_t)(pair & 0xffu);
                tile[c + 2 * i + 1][r] = (uint8_t)(pair >> 8);
            }
        }
    }
    __syncthreads();
    const int f = tid >> 2, c = (tid & 3) * 16, row = r0 + c;
    if (row >= rows) return;
    uint8_t* dst = out + (size_t)(f0 + f) * rows + row;
    if ((rows & 15) == 0) {
        *(uint4*)dst = *(const uint4*)&tile[f][c];
    } else {
        const int n = min(16, rows - row);
        for (int i = 0; i < n; ++i) dst[i] = tile[f][c + i];
    }
}

// out[(h * 272 + p) * 128 + d] = in[p * 1024 + h * 128 + d], 8 halves a thread.
__global__ __launch_bounds__(256) void pack_position_heads_kernel(const uint4* __restrict__ in, uint4* __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= kPosRows * kModel / 8) return;
    const int p = i >> 7, h = (i >> 4) & 7, d8 = i & 15;
    out[((h * kPosRows + p) * kHeadW >> 3) + d8] = in[i];
}

struct ShortArgs {
    const uint16_t *q, *k, *v, *pos, *bu, *bv;
    uint16_t* out;
    int rows, padded, valid, left, right;
};

__global__ __launch_bounds__(256) void attention_short_kernel(ShortArgs a) {
    __shared__ float scores[4][kMaxKeys + 3];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int query = blockIdx.x * 4 + wave, head = blockIdx.y;
    if (query >= a.padded) return;
    uint16_t* o = a.out + (size_t)query * kModel + head * kHeadW + 2 * lane;
    if (query >= a.rows || query >= a.valid) {
        *(uint32_t*)o = 0u;
        return;
    }
    float* sc = scores[wave];
    const int first = max(0, query - a.left), last = min(a.valid - 1, query + a.right);
    const int count = last - first + 1;
    const int grp = lane >> 4, gl = lane & 15;
    // (q + u) and (q + v) of this lane's 8 dimensions
    float qu[8], qv[8];
    {
        const int d = head * kHeadW + 8 * gl;
        const uint4 q4 = *(const uint4*)(a.q + (size_t)query * kModel + d);
        const uint4 u4 = *(const uint4*)(a.bu + d);
        const uint4 v4 = *(const uint4*)(a.bv + d);
        const uint32_t qw[4] = {q4.x, q4.y, q4.z, q4.w}, uw[4] = {u4.x, u4.y, u4.z, u4.w}, vw[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float q0 = h2f((uint16_t)(qw[i] & 0xffffu)), q1 = h2f((uint16_t)(qw[i] >> 16));
            qu[2 * i] = q0 + h2f((uint16_t)(uw[i] & 0xffffu));
            qu[2 * i + 1] = q1 + h2f((uint16_t)(uw[i] >> 16));
            qv[2 * i] = q0 + h2f((uint16_t)(vw[i] & 0xffffu));
            qv[2 * i + 1] = q1 + h2f((uint16_t)(vw[i] >> 16));
        }
    }
    // scores, four keys a pass; the K and position rows of the next two passes are in flight
    auto load = [&](int s0, uint4& k4, uint4& p4) {
        const int key_row = first + min(s0 + grp, count - 1);
        const int prow = a.left - query + key_row;
        k4 = *(const uint4*)(a.k + (size_t)key_row * kModel + head * kHeadW + 8 * gl);
        p4 = *(const uint4*)(a.pos + ((size_t)head * kPosRows + prow) * kHeadW + 8 * gl);
    };
    uint4 kb[3], pb[3];
    load(0, kb[0], pb[0]);
    load(4, kb[1], pb[1]);
    for (int s0 = 0; s0 < count; s0 += 12) {
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            const int base = s0 + 4 * u;
            if (base >= count) break;
            load(base + 8, kb[(u + 2) % 3], pb[(u + 2) % 3]);
            const uint32_t kw[4] = {kb[u].x, kb[u].y, kb[u].z, kb[u].w}, pw[4] = {pb[u].x, pb[u].y, pb[u].z, pb[u].w};
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s = __builtin_fmaf(qu[2 * i], h2f((uint16_t)(kw[i] & 0xffffu)), s);
                s = __builtin_fmaf(qv[2 * i], h2f((uint16_t)(pw[i] & 0xffffu)), s);
                s = __builtin_fmaf(qu[2 * i + 1], h2f((uint16_t)(kw[i] >> 16)), s);
                s = __builtin_fmaf(qv[2 * i + 1], h2f((uint16_t)(pw[i] >> 16)), s);
            }
            s = row_sum16(s);
            const int slot = base + grp;
            if (gl == 0 && slot < count) sc[slot] = s * 0.08838834764831845f;
        }
    }
    wave_fence();
    float mx = -3.402823466e38f;
    for (int slot = lane; slot < count; slot += 64) mx = __builtin_fmaxf(mx, sc[slot]);
    mx = wave_max(mx);
    float den = 0.0f;
    for (int slot = lane; slot < count; slot += 64) {
        const float e = __expf(sc[slot] - mx);  // the reference's fast-math exponential (build.rs:68-73)
        sc[slot] = e;
        den += e;
    }
    den = sum_desc<64>(den);  // xor 32, ..., 1
    // probabilities, each divided once (the reference divides per lane and key: same value)
    for (int slot = lane; slot < count; slot += 64) sc[slot] = sc[slot] / den;
    wave_fence();
    float c0 = 0.0f, c1 = 0.0f;
    const uint16_t* vp = a.v + (size_t)first * kModel + head * kHeadW + 2 * lane;
    int slot = 0;
    for (; slot + 8 <= count; slot += 8) {  // eight V rows in flight
        uint32_t v2[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v2[i] = *(const uint32_t*)(vp + (size_t)(slot + i) * kModel);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float w = sc[slot + i];
            c0 = __builtin_fmaf(w, h2f((uint16_t)(v2[i] & 0xffffu)), c0);
            c1 = __builtin_fmaf(w, h2f((uint16_t)(v2[i] >> 16)), c1);
        }
    }
    for (; slot < count; ++slot) {
        const float w = sc[slot];
        const uint32_t v2 = *(const uint32_t*)(vp + (size_t)slot * kModel);
        c0 = __builtin_fmaf(w, h2f((uint16_t)(v2 & 0xffffu)), c0);
        c1 = __builtin_fmaf(w, h2f((uint16_t)(v2 >> 16)), c1);
    }
    *(uint32_t*)o = (uint32_t)f2h(c0) | ((uint32_t)f2h(c1) << 16);
}

}  // namespace

void launch_quantize_fp8_transpose(const uint16_t* in, uint8_t* out, int rows, float inverse_scale, hipStream_t s) {
    if (rows <= 0) return;
    quantize_fp8_transpose_kernel<<<dim3(kModel / 64, (rows + 63) / 64), 256, 0, s>>>(in, out, rows, inverse_scale);
}

void launch_pack_position_heads(const uint16_t* in, uint16_t* out, hipStream_t s) {
    const int chunks = kPosRows * kModel / 8;
    pack_position_heads_kernel<<<(chunks + 255) / 256, 256, 0, s>>>((const uint4*)in, (uint4*)out);
}

void launch_local_attention_short(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* pos,
                                  const uint16_t* bu, const uint16_t* bv, uint16_t* out, int rows, int padded_rows,
                                  int valid_rows, int left, int right, hipStream_t s) {
    ShortArgs a{q, k, v, pos, bu, bv, out, rows, padded_rows, valid_rows, left, right};
    attention_short_kernel<<<dim3((padded_rows + 3) / 4, kHeadsN), 256, 0, s>>>(a);
}

}  // namespace pk
