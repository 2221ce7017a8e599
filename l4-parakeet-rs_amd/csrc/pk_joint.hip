// Batch-1 TDT joint (decoder.cu:690-759): per frame t,
//   score[o] = bias[o] + w_scale[o] * sum_k W[o,k] * relu(enc[t,k] + pred[k])
// then the greedy token / duration decision.  The GEMV is HBM/L2-bound: one
// wave64 per output row, each lane streaming 16 bytes (int8) or 16 bytes of
// fp16 per pass, the activation vector staged once per block in LDS.
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

int launch_joint(const void* w, int w_int8, const float* w_scales, const float* bias, const void* enc, const float* pred,
                 float* scores, int* decision, int outputs, int hidden, int token_outputs, int durations, int steps,
                 int enc_stride, hipStream_t s) {
    if (steps == 0) return 0;
    const dim3 grid((outputs + 3) / 4, steps);
    if (w_int8)
        joint_scores_kernel<true><<<grid, 256, 0, s>>>(w, w_scales, bias, (const uint16_t*)enc, pred, scores, outputs, hidden, enc_stride);
    else
        joint_scores_kernel<false><<<grid, 256, 0, s>>>(w, w_scales, bias, (const uint16_t*)enc, pred, scores, outputs, hidden, enc_stride);
    if (decision) joint_decide_kernel<<<steps, 256, 0, s>>>(scores, decision, outputs, token_outputs, durations);
    return 0;
}

}  // namespace pk
