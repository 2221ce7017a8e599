// Activation quantizers, load-time weight packers and LayerNorm producers.
// All are HBM-bound byte work: one 256-thread block per row for the per-row
// kinds, 8 elements (16 bytes of fp16) per thread for the elementwise kinds.
#include "pk_kernels.hpp"

namespace pk {

// linear.cu:537-547, encoder.cu:549-559: e4m3(f16 * inverse_scale).
__global__ void quantize_fp8_static_kernel(const uint16_t* __restrict__ in, uint8_t* __restrict__ out,
                                           float inverse_scale, size_t elements) {
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i + 8 <= elements) {
        const uint4 raw = *(const uint4*)(in + i);
        const uint16_t* h = (const uint16_t*)&raw;
        uint32_t w0 = e4m3x2(h2f(h[0]) * inverse_scale, h2f(h[1]) * inverse_scale) |
                      (e4m3x2(h2f(h[2]) * inverse_scale, h2f(h[3]) * inverse_scale) << 16);
        uint32_t w1 = e4m3x2(h2f(h[4]) * inverse_scale, h2f(h[5]) * inverse_scale) |
                      (e4m3x2(h2f(h[6]) * inverse_scale, h2f(h[7]) * inverse_scale) << 16);
        *(uint2*)(out + i) = uint2{w0, w1};
    } else {
        for (size_t j = i; j < elements; ++j) out[j] = e4m3(h2f(in[j]) * inverse_scale);
    }
}

// linear.cu:549-560: rne(clamp(f16 * inverse_scale, +-127)).
__global__ void quantize_int8_static_kernel(const uint16_t* __restrict__ in, int8_t* __restrict__ out,
                                            float inverse_scale, size_t elements) {
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    const size_t end = i + 8 <= elements ? i + 8 : elements;
    for (size_t j = i; j < end; ++j) {
        const float s = __builtin_fminf(127.0f, __builtin_fmaxf(-127.0f, h2f(in[j]) * inverse_scale));
        out[j] = (int8_t)__builtin_rintf(s);
    }
}

__device__ __forceinline__ float block_max_256(float v, float* red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    __syncthreads();
    return r;
}

// Dynamic per-row quantization of fp16 rows [rows x k] (k % 8 == 0).
//   kind 0: FP8,  scale = max|x| / 448 (encoder.cu:1129-1180, :264-292)
//   kind 1: INT8, scale = max|x| / 127 (per-token dynamic INT8)
//   kind 2: INT4, scale = max(max(x/7, -x/8)), nibble pairs (encoder.cu:264-290)
// Scale is 1 for a row without a positive maximum; rows >= valid_rows are
// written as zeros with scale 1 (padding rows, encoder.cu:226-237).
template <int kind>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const uint16_t* __restrict__ in, uint8_t* __restrict__ out,
                                                            float* __restrict__ scales, int k, int valid_rows) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const uint16_t* x = in + (size_t)row * k;
    const int out_row = kind == 2 ? k / 2 : k;
    uint8_t* o = out + (size_t)row * out_row;
    if (row >= valid_rows) {
        for (int i = threadIdx.x * 8; i < out_row; i += 256 * 8) {
            if (i + 8 <= out_row) *(uint2*)(o + i) = uint2{0, 0};
            else for (int j = i; j < out_row; ++j) o[j] = 0;
        }
        if (threadIdx.x == 0) scales[row] = 1.0f;
        return;
    }
    float m = 0.0f;
    for (int i = threadIdx.x * 8; i < k; i += 256 * 8) {
        const uint4 raw = *(const uint4*)(x + i);
        const uint16_t* h = (const uint16_t*)&raw;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float v = h2f(h[j]);
            m = kind == 2 ? __builtin_fmaxf(m, __builtin_fmaxf(v / 7.0f, -v / 8.0f)) : __builtin_fmaxf(m, __builtin_fabsf(v));
        }
    }
    m = block_max_256(m, red);
    const float scale = m > 0.0f ? (kind == 0 ? m / 448.0f : (kind == 1 ? m / 127.0f : m)) : 1.0f;
    if (threadIdx.x == 0) scales[row] = scale;
    for (int i = threadIdx.x * 8; i < k; i += 256 * 8) {
        const uint4 raw = *(const uint4*)(x + i);
        const uint16_t* h = (const uint16_t*)&raw;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = h2f(h[j]) / scale;
        if constexpr (kind == 0) {
            const uint32_t w0 = e4m3x2(v[0], v[1]) | (e4m3x2(v[2], v[3]) << 16);
            const uint32_t w1 = e4m3x2(v[4], v[5]) | (e4m3x2(v[6], v[7]) << 16);
            *(uint2*)(o + i) = uint2{w0, w1};
        } else if constexpr (kind == 1) {
            uint32_t w[2] = {0, 0};
#pragma unroll
            for (int j = 0; j < 8; ++j) w[j >> 2] |= ((uint32_t)rne_clamp(v[j], -127, 127) & 255u) << (8 * (j & 3));
            *(uint2*)(o + i) = uint2{w[0], w[1]};
        } else {
            uint32_t w = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) w |= ((uint32_t)rne_clamp(v[j], -8, 7) & 15u) << (4 * j);
            *(uint32_t*)(o + i / 2) = w;
        }
    }
}

// Per-row weight packers (load-time derivation, encoder.rs:361-422 and
// quant_benchmark.rs:779-829), rows of fp16 [n x k]:
//   kind 0: FP8  scale = max|w| / 448 (1 for zero rows)
//   kind 1: INT8 scale = max|w| / 127 (1 for zero rows)
//   kind 2: INT4 scale = max(max(w/7, -w/8)) folded from 0; zero rows keep
//           scale 0 and pack to zero bytes (encoder.rs:378-407).
template <int kind>
__global__ __launch_bounds__(256) void pack_rows_kernel(const uint16_t* __restrict__ w, uint8_t* __restrict__ out,
                                                        float* __restrict__ scales, int k) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const uint16_t* x = w + (size_t)row * k;
    float m = 0.0f;
    for (int i = threadIdx.x; i < k; i += 256) {
        const float v = h2f(x[i]);
        m = kind == 2 ? __builtin_fmaxf(m, __builtin_fmaxf(v / 7.0f, -v / 8.0f)) : __builtin_fmaxf(m, __builtin_fabsf(v));
    }
    m = block_max_256(m, red);
    const float scale = kind == 2 ? m : (m > 0.0f ? m / (kind == 0 ? 448.0f : 127.0f) : 1.0f);
    if (threadIdx.x == 0) scales[row] = scale;
    if constexpr (kind == 2) {
        for (int j = threadIdx.x; j < k / 2; j += 256) {
            const int a = rne_clamp(h2f(x[2 * j]) / scale, -8, 7);
            const int b = rne_clamp(h2f(x[2 * j + 1]) / scale, -8, 7);
            out[(size_t)row * (k / 2) + j] = (uint8_t)((a & 15) | ((b & 15) << 4));
        }
    } else {
        for (int i = threadIdx.x; i < k; i += 256) {
            const float v = h2f(x[i]) / scale;
            out[(size_t)row * k + i] = kind == 0 ? e4m3(v) : (uint8_t)(int8_t)rne_clamp(v, -127, 127);
        }
    }
}

// Group-wise asymmetric INT4 packer, one thread per (row, 128-K group):
// lo = min(0, min w), hi = max(0, max w), s = fp16((hi - lo) / 15) (1 if not
// positive), z = clamp(rne(-lo / s), 0, 15), q = clamp(rne(w / s) + z, 0, 15).
// Device layout: word j of a row holds k = 8j .. 8j+7; byte b of the word
// holds k = 8j+b in its low nibble and k = 8j+4+b in its high nibble, so
// (w & 0x0f0f0f0f) and (w >> 4 & 0x0f0f0f0f) are the eight levels in k order.
__global__ void pack_g128_kernel(const uint16_t* __restrict__ w, uint32_t* __restrict__ q, uint16_t* __restrict__ scales,
                                 uint16_t* __restrict__ zeros, int n, int k) {
    const int groups = k / 128;
    const int id = blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n * groups) return;
    const int row = id / groups, g = id - row * groups;
    const uint16_t* x = w + (size_t)row * k + g * 128;
    float lo = 0.0f, hi = 0.0f;
    for (int i = 0; i < 128; ++i) {
        const float v = h2f(x[i]);
        lo = __builtin_fminf(lo, v);
        hi = __builtin_fmaxf(hi, v);
    }
    float s = round_f16((hi - lo) / 15.0f);
    if (!(s > 0.0f)) s = 1.0f;
    const int z = rne_clamp(-lo / s, 0, 15);
    scales[id] = f2h(s);
    zeros[id] = f2h((float)z);
    for (int j = 0; j < 16; ++j) {
        uint32_t word = 0;
        for (int i = 0; i < 8; ++i) {
            int level = rne_clamp(h2f(x[8 * j + i]) / s, -64, 64) + z;
            level = level < 0 ? 0 : (level > 15 ? 15 : level);
            word |= (uint32_t)level << (8 * (i & 3) + 4 * (i >> 2));
        }
        q[(size_t)row * (k / 8) + g * 16 + j] = word;
    }
}

// LayerNorm over 1024 features + dynamic per-row FP8 / INT4 quantization
// (encoder.cu:211-306).  The sums keep the reference's reduction shape:
// thread t folds x[t], x[t+256], x[t+512], x[t+768]; lanes 0..31 combine
// (t, t+128), (t+64, t+192), (t+32, t+160), (t+96, t+224) as
// ((s0 + s1) + (s2 + s3)) and a shuffle-down tree over 32 lanes finishes
// (encoder.cu:36-54).  inverse_std = 1 / sqrtf(.) correctly rounded.
__device__ __forceinline__ float tree_sum_256(float v, float* part) {
    const int t = threadIdx.x;
    part[t] = v;
    __syncthreads();
    float r = 0.0f;
    if (t < 64) {
        const int l = t & 31;
        const float s0 = part[l] + part[l + 128];
        const float s1 = part[l + 64] + part[l + 192];
        const float s2 = part[l + 32] + part[l + 160];
        const float s3 = part[l + 96] + part[l + 224];
        r = (s0 + s1) + (s2 + s3);
        for (int off = 16; off > 0; off >>= 1) {
            const float o = __shfl_down(r, off, 32);
            r = (l + off < 32) ? r + o : r;
        }
        if (t == 0) part[256] = r;
    }
    __syncthreads();
    r = part[256];
    __syncthreads();
    return r;
}

template <bool kInt4>
__global__ __launch_bounds__(256) void layer_norm_quantize_kernel(const uint16_t* __restrict__ in, const uint16_t* __restrict__ gamma,
                                                                  const uint16_t* __restrict__ beta, uint8_t* __restrict__ out,
                                                                  float* __restrict__ scales, uint16_t* __restrict__ normalized,
                                                                  int rows, float epsilon) {
    __shared__ float part[257];
    __shared__ float red[4];
    const int row = blockIdx.x, t = threadIdx.x;
    if (row >= rows) {
        for (int f = t; f < 1024; f += 256) {
            if (kInt4) { if ((f & 1) == 0) out[((size_t)row * 1024 + f) / 2] = 0; }
            else out[(size_t)row * 1024 + f] = 0;
            if (normalized) normalized[(size_t)row * 1024 + f] = 0;
        }
        if (t == 0) scales[row] = 1.0f;
        return;
    }
    float v[4];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = h2f(in[(size_t)row * 1024 + t + 256 * i]);
        sum += v[i];
    }
    const float mean = tree_sum_256(sum, part) / 1024.0f;
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float d = v[i] - mean;
        sq += d * d;
    }
    const float inverse_std = 1.0f / sqrtf(tree_sum_256(sq, part) / 1024.0f + epsilon);
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int f = t + 256 * i;
        const float y = (v[i] - mean) * inverse_std * h2f(gamma[f]) + h2f(beta[f]);
        const uint16_t h = f2h(y);
        if (normalized) normalized[(size_t)row * 1024 + f] = h;
        v[i] = h2f(h);
        m = kInt4 ? __builtin_fmaxf(m, __builtin_fmaxf(v[i] / 7.0f, -v[i] / 8.0f)) : __builtin_fmaxf(m, __builtin_fabsf(v[i]));
    }
    m = block_max_256(m, red);
    const float scale = m > 0.0f ? (kInt4 ? m : m / 448.0f) : 1.0f;
    if (t == 0) scales[row] = scale;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int f = t + 256 * i;
        if constexpr (kInt4) {
            const int q = rne_clamp(v[i] / scale, -8, 7);
            const int other = __shfl_xor(q, 1, 64);
            if ((t & 1) == 0) out[((size_t)row * 1024 + f) / 2] = (uint8_t)((q & 15) | ((other & 15) << 4));
        } else {
            out[(size_t)row * 1024 + f] = e4m3(v[i] / scale);
        }
    }
}

// ---- launchers -------------------------------------------------------------

// Q4_K superblocks -> fp16 [n x k] (linear.cu:459-472): one thread per 8
// consecutive values of one 32-value group.
__global__ __launch_bounds__(256) void q4k_dequant_kernel(const uint8_t* __restrict__ blocks, uint16_t* __restrict__ out, int n,
                                                          int k) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t per_row = (size_t)k / 8;
    if (idx >= (size_t)n * per_row) return;
    const size_t row = idx / per_row;
    const int t = (int)(idx - row * per_row) * 8;
    const uint8_t* blk = blocks + (row * (size_t)(k / 256) + (size_t)(t >> 8)) * 144;
    const int v = t & 255, group = v >> 5;
    const uint4 h = *(const uint4*)blk;
    const uint2 q = *(const uint2*)(blk + 16 + (group >> 1) * 32 + (v & 31));
    float a, b;
    q4k_coeffs(h, group, a, b);
    const int sh = (group & 1) * 4;
    *(uint4*)(out + row * (size_t)k + t) = q4k_decode8((q.x >> sh) & 0x0f0f0f0fu, (q.y >> sh) & 0x0f0f0f0fu, a, b);
}

int launch_quantize_static(const void* in, void* out, float inverse_scale, size_t elements, bool int8, hipStream_t s) {
    if (elements == 0) return 0;
    const size_t threads = (elements + 7) / 8;
    const unsigned grid = (unsigned)((threads + 255) / 256);
    if (int8) quantize_int8_static_kernel<<<grid, 256, 0, s>>>((const uint16_t*)in, (int8_t*)out, inverse_scale, elements);
    else quantize_fp8_static_kernel<<<grid, 256, 0, s>>>((const uint16_t*)in, (uint8_t*)out, inverse_scale, elements);
    return 0;
}

int launch_quantize_rows(int kind, const void* in, void* out, float* scales, int rows, int valid_rows, int k, hipStream_t s) {
    if (rows == 0) return 0;
    if (kind == 0) quantize_rows_kernel<0><<<rows, 256, 0, s>>>((const uint16_t*)in, (uint8_t*)out, scales, k, valid_rows);
    else if (kind == 1) quantize_rows_kernel<1><<<rows, 256, 0, s>>>((const uint16_t*)in, (uint8_t*)out, scales, k, valid_rows);
    else quantize_rows_kernel<2><<<rows, 256, 0, s>>>((const uint16_t*)in, (uint8_t*)out, scales, k, valid_rows);
    return 0;
}

int launch_pack_rows(int kind, const void* w, void* out, float* scales, int n, int k, hipStream_t s) {
    if (n == 0) return 0;
    if (kind == 0) pack_rows_kernel<0><<<n, 256, 0, s>>>((const uint16_t*)w, (uint8_t*)out, scales, k);
    else if (kind == 1) pack_rows_kernel<1><<<n, 256, 0, s>>>((const uint16_t*)w, (uint8_t*)out, scales, k);
    else pack_rows_kernel<2><<<n, 256, 0, s>>>((const uint16_t*)w, (uint8_t*)out, scales, k);
    return 0;
}

int launch_pack_g128(const void* w, uint32_t* q, uint16_t* scales, uint16_t* zeros, int n, int k, hipStream_t s) {
    const int total = n * (k / 128);
    if (total == 0) return 0;
    pack_g128_kernel<<<(total + 255) / 256, 256, 0, s>>>((const uint16_t*)w, q, scales, zeros, n, k);
    return 0;
}

int launch_layer_norm_quantize(bool int4, const void* in, const void* gamma, const void* beta, void* out, float* scales,
                               void* normalized, int rows, int padded_rows, float epsilon, hipStream_t s) {
    if (padded_rows == 0) return 0;
    if (int4)
        layer_norm_quantize_kernel<true><<<padded_rows, 256, 0, s>>>((const uint16_t*)in, (const uint16_t*)gamma, (const uint16_t*)beta,
                                                                      (uint8_t*)out, scales, (uint16_t*)normalized, rows, epsilon);
    else
        layer_norm_quantize_kernel<false><<<padded_rows, 256, 0, s>>>((const uint16_t*)in, (const uint16_t*)gamma, (const uint16_t*)beta,
                                                                       (uint8_t*)out, scales, (uint16_t*)normalized, rows, epsilon);
    return 0;
}

int launch_q4k_dequant(const uint8_t* blocks, uint16_t* out, int n, int k, hipStream_t s) {
    const size_t threads = (size_t)n * (k / 8);
    if (threads == 0) return 0;
    hipLaunchKernelGGL(q4k_dequant_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, blocks, out, n, k);
    return 0;
}

}  // namespace pk
