// SOFT_MAX f32: dst = softmax(x * scale + slope * mask) over each row.
//
// Semantics: ggml_compute_forward_soft_max_f32 (ggml-cpu/ops.cpp:5519-5629):
// mask row = row index (broadcast over dims 2/3 by modulo), ALiBi slope per
// head (dim 2) when max_bias > 0, max-subtracted exp, sum, scale by 1/sum.
// One workgroup (256 lanes) per row; row staged in registers (up to 16 values
// per lane) or re-read from global for longer rows.
#include "common.h"
#include "kernels.h"

namespace gq {

namespace {

__device__ float block_reduce(float v, bool is_max, float* red) {
    v = is_max ? xor_max<64>(v) : xor_sum<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    return r;
}

__global__ __launch_bounds__(256) void k_soft_max(SoftmaxArgs a, float m0, float m1, uint32_t n_head_log2) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const int64_t i1 = row % a.nrows;
    const int64_t i2 = (row / a.nrows) % a.n2;
    const int64_t i3 = row / (a.nrows * a.n2);
    const float* x = reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(a.x) + i1 * a.xnb1 +
                                                    i2 * a.xnb2 + i3 * a.xnb3);
    float* y = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(a.y) + i1 * a.ynb1 + i2 * a.ynb2 + i3 * a.ynb3);
    const uint8_t* mrow = a.mask ? reinterpret_cast<const uint8_t*>(a.mask) + i1 * a.mnb1 +
                                       (i2 % a.mne2) * a.mnb2 + (i3 % a.mne3) * a.mnb3
                                 : nullptr;
    float slope = 1.0f;
    if (a.max_bias > 0.0f) {
        const uint32_t h = (uint32_t)i2;
        slope = h < n_head_log2 ? powf(m0, (float)(h + 1)) : powf(m1, (float)(2 * (h - n_head_log2) + 1));
    }
    float mx = -INFINITY;
    for (int64_t c = threadIdx.x; c < a.ncols; c += blockDim.x) {
        float v = x[c] * a.scale;
        if (mrow) {
            const float mv = a.mask_f16 ? h2f(reinterpret_cast<const uint16_t*>(mrow)[c])
                                        : reinterpret_cast<const float*>(mrow)[c];
            v += slope * mv;
        }
        y[c] = v;
        mx = fmaxf(mx, v);
    }
    mx = block_reduce(mx, true, red);
    float sum = 0.0f;
    for (int64_t c = threadIdx.x; c < a.ncols; c += blockDim.x) {
        const float e = expf(y[c] - mx);
        y[c] = e;
        sum += e;
    }
    sum = block_reduce(sum, false, red);
    const float inv = 1.0f / sum;
    for (int64_t c = threadIdx.x; c < a.ncols; c += blockDim.x) y[c] *= inv;
}

}  // namespace

int soft_max(const SoftmaxArgs& a, hipStream_t s) {
    const int64_t rows = a.nrows * a.n2 * a.n3;
    if (rows == 0 || a.ncols == 0) return GQ_OK;
    const uint32_t n_head = (uint32_t)a.n2;
    const uint32_t n_head_log2 = 1u << (uint32_t)floor(log2((double)n_head));
    const float m0 = powf(2.0f, -(a.max_bias) / n_head_log2);
    const float m1 = powf(2.0f, -(a.max_bias / 2.0f) / n_head_log2);
    hipLaunchKernelGGL(k_soft_max, dim3((unsigned)rows), dim3(256), 0, s, a, m0, m1, n_head_log2);
    return check_hip(hipGetLastError(), "soft_max launch");
}

}  // namespace gq
