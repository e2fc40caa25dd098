// Activation and weight quantizers.
//
// Activation: the rule of ggml's x86 quantize_row_q8_0
// (third_party/ggml/src/ggml-cpu/arch/x86/quants.c:302-398), which the CPU
// backend applies to MUL_MAT's src1 (ggml-cpu/ggml-cpu.c:1322-1357):
//   amax = max|x|, d = fp16_rne(amax / 127), id = amax ? 127 / amax : 0,
//   q = saturate_int8(round_half_even(x * id)).
// Four lanes own one 32-element block (8 elements each, two 16-byte loads);
// amax is exchanged with two xor shuffles (quant8_block, common.h). The GEMV
// path runs the same code inside its own kernel (quantize_rows_to_act).
//
// Weights: ggmlc's compile-time quantizers (python/ggmlc/quantization/
// quantize.py:10-47 Q8_0, :65-107 Q4_0) with numpy float32 semantics, one
// lane per block. They only build device-resident weights for tests/benches.
#include "common.h"
#include "kernels.h"

// x * id and x / scale must round once each, exactly as the CPU code does.
#pragma clang fp contract(off)

namespace gq {

enum ActOut { OUT_BLOCKS = 0, OUT_F16 = 2 };

// One lane per 8 elements, 4 lanes per block (quant8_block in common.h).
template <int MODE, bool VEC>
__global__ __launch_bounds__(256) void k_quantize_act(const float* __restrict__ x, int64_t nrows,
                                                      int64_t K, int64_t x_stride,
                                                      uint8_t* __restrict__ y, int64_t y_stride,
                                                      const float* __restrict__ rs) {
    const int64_t nb = K / QK;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gid >> 2;
    const int part = (int)(gid & 3);
    const bool valid = blk < nrows * nb;
    const int64_t m = valid ? blk / nb : 0;
    const int64_t b = valid ? blk - m * nb : 0;

    float v[8];
    load8<VEC>(x + m * x_stride + b * QK + part * 8, valid, v);
    int q[8];
    uint16_t dh;
    int qsum;
    quant8_block(v, q, dh, qsum);
    if (!valid) return;

    if (MODE == OUT_BLOCKS) {
        uint8_t* blkp = y + (m * nb + b) * Q8_BYTES;
        if (part == 0) *reinterpret_cast<uint16_t*>(blkp) = dh;
        uint16_t* qp = reinterpret_cast<uint16_t*>(blkp + 2 + part * 8);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            qp[i] = (uint16_t)((q[2 * i] & 0xff) | ((q[2 * i + 1] & 0xff) << 8));
    } else {  // OUT_F16: the GEMM's A operand, d * q / r as fp16 hi (at k) + lo (at K + k) of the row
        uint4 hi, lo;
        split_dq8(q, dh, 1.0f / rs[m], hi, lo);  // r a power of two: 1 / r exact
        uint16_t* row = reinterpret_cast<uint16_t*>(y) + m * y_stride + b * QK + part * 8;
        *reinterpret_cast<uint4*>(row) = hi;
        *reinterpret_cast<uint4*>(row + K) = lo;
    }
}

// The row scales r of the fp16 pairs (row_pow2) for rows quantized block by block: one
// workgroup per row takes max|x| over the row; fp16(max / 127) is the row's largest block
// scale, since the division and the rounding are monotone.
__global__ __launch_bounds__(256) void k_row_scale(const float* __restrict__ x, int64_t K, int64_t x_stride,
                                                   float* __restrict__ rs) {
    __shared__ float red[4];
    const float* xr = x + (int64_t)blockIdx.x * x_stride;
    float amax = 0.0f;
    for (int64_t k = threadIdx.x; k < K; k += 256) amax = fmaxf(amax, fabsf(xr[k]));
    amax = xor_max<64>(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    if (threadIdx.x == 0)
        rs[blockIdx.x] = row_pow2(h2f(f2h(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) / 127.0f)));
}

template <int MODE>
static int launch_quant(const float* x, int64_t nrows, int64_t K, int64_t x_stride, void* y,
                        int64_t y_stride, hipStream_t s, const float* rs = nullptr) {
    const int64_t threads = nrows * (K / QK) * 4;
    if (threads == 0) return GQ_OK;
    const bool vec = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && (x_stride % 4 == 0);
    const dim3 grid((unsigned)cdiv(threads, 256));
    if (vec)
        hipLaunchKernelGGL((k_quantize_act<MODE, true>), grid, dim3(256), 0, s, x, nrows, K, x_stride,
                           (uint8_t*)y, y_stride, rs);
    else
        hipLaunchKernelGGL((k_quantize_act<MODE, false>), grid, dim3(256), 0, s, x, nrows, K, x_stride,
                           (uint8_t*)y, y_stride, rs);
    return check_hip(hipGetLastError(), "quantize launch");
}

int quantize_q8_0_blocks(const float* x, int64_t nrows, int64_t K, int64_t x_stride, void* y,
                         hipStream_t s) {
    return launch_quant<OUT_BLOCKS>(x, nrows, K, x_stride, y, 0, s);
}

int quantize_q8_0_f16(const float* x, int64_t nrows, int64_t K, int64_t x_stride, uint16_t* y,
                      int64_t y_stride_elems, float* rs, hipStream_t s) {
    if (nrows == 0 || K == 0) return GQ_OK;
    hipLaunchKernelGGL(k_row_scale, dim3((unsigned)nrows), dim3(256), 0, s, x, K, x_stride, rs);
    if (int rc = check_hip(hipGetLastError(), "row scale launch")) return rc;
    return launch_quant<OUT_F16>(x, nrows, K, x_stride, y, y_stride_elems, s, rs);
}

// ---- fused activation prologue of the GEMM path ----------------------------------
// One workgroup per activation row: v = x (+ d, or + (d + d2), stored to `sum`), then RMS_NORM
// (v * scale, the sum of squares in the order of k_rms_norm) or SWIGLU of the row's
// halves (silu(x[c]) * x[K + c], the arithmetic of k_swiglu), then the fp16(d * q)
// of quantize_row_q8_0 — the bits of ADD -> RMS_NORM -> quantize (or SWIGLU ->
// quantize) run one by one — written as the exact fp16 pair hi (row[k]) + lo (row[K + k])
// of d * q / r, with the row scale r (row_pow2 of the row's largest block scale: 1 below
// amax ~65500) stored to rs[m] for the GEMM's epilogue. Thread t holds elements
// c * 2048 + 8t.. of every 2048-wide chunk c in registers (K <= PREP_MAX_K).
constexpr int PREP_CH = PREP_MAX_K / 2048;

// CH > 0: the launch has exactly CH chunks (straight-line code the compiler can
// interleave); CH = 0: up to PREP_CH chunks, the ones past K skipped. I8: the int8 layout
// of gemm_i8 (quants, scale, block sum per (block, row)) instead of the fp16 pair. SPLIT (I8
// without RMS_NORM, CH = 1): one workgroup per (row, 2048-element chunk blockIdx.y), since
// nothing then spans the row; every piece gets the operations of the one-workgroup launch.
template <bool VEC, int CH, bool I8 = false, bool SPLIT = false>
__global__ __launch_bounds__(256) void k_act_prep(ActPrep a, uint16_t* __restrict__ y, int64_t y_stride,
                                                  float* __restrict__ rs) {
    static_assert(!SPLIT || (I8 && CH == 1), "chunk workgroups for the int8 layout");
    constexpr int NC = CH ? CH : PREP_CH;
    __shared__ double red[4];
    __shared__ float redf[4];
    const int64_t m = blockIdx.x;
    const int nb = (int)(a.K / QK);
    const float* xr = a.x + m * a.xs;
    const int c0 = SPLIT ? (int)blockIdx.y : 0;  // first chunk of the workgroup
    float v[NC][8];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int t = (c0 + c) * 256 + (int)threadIdx.x;  // 8-element piece
        const bool valid = (t >> 2) < nb;
        if (!CH && c * 2048 >= a.K) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[c][i] = 0.0f;
            continue;
        }
        if (a.glu) {
            float u[8];
            load8<VEC>(xr + (int64_t)t * 8, valid, v[c]);
            load8<VEC>(xr + a.K + (int64_t)t * 8, valid, u);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[c][i] = swiglu_f(v[c][i], u[i]);
        } else {
            load8<VEC>(xr + (int64_t)t * 8, valid, v[c]);
            if (a.d) {
                float w[8];
                load8<VEC>(a.d + m * a.ds + (int64_t)t * 8, valid, w);
                if (a.d2) {  // a product left in two halves: their sum first
                    float w2[8];
                    load8<VEC>(a.d2 + m * a.ds + (int64_t)t * 8, valid, w2);
#pragma unroll
                    for (int i = 0; i < 8; ++i) w[i] = w[i] + w2[i];
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) v[c][i] = v[c][i] + w[i];
                if (a.sum && valid) {
                    float* o = a.sum + m * a.ss + (int64_t)t * 8;
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = v[c][i];
                }
            }
        }
    }
    if (!SPLIT && a.rms) {
        double sq = 0.0;
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (CH || c * 2048 < a.K) sq = sumsq8(v[c], sq);
        const float sc = rms_scale(block_sum_d(sq, red), a.K, a.eps);
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) v[c][i] = v[c][i] * sc;
    }
    if constexpr (I8) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (!CH && c * 2048 >= a.K) break;  // uniform: whole chunks past K
            const int t = (c0 + c) * 256 + (int)threadIdx.x;
            int q[8];
            uint16_t dh;
            int qsum;
            quant8_block(v[c], q, dh, qsum);  // all lanes: pieces past K quantize zeros
            if ((t >> 2) >= nb) continue;
            uint8_t* yb = reinterpret_cast<uint8_t*>(y);
            const int64_t e = (int64_t)(t >> 2) * 16 + m;  // (block, row)
            uint32_t w0 = 0, w1 = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                w0 |= (uint32_t)(q[i] & 0xff) << (8 * i);
                w1 |= (uint32_t)(q[4 + i] & 0xff) << (8 * i);
            }
            *reinterpret_cast<uint2*>(yb + e * 32 + (t & 3) * 8) = make_uint2(w0, w1);
            if ((t & 3) == 0) {
                *reinterpret_cast<float*>(yb + (int64_t)nb * 512 + e * 4) = h2f(dh);
                *reinterpret_cast<int*>(yb + (int64_t)nb * 576 + e * 4) = qsum;
            }
        }
    } else {
        // quantize every chunk first: the row's largest block scale sets r before any
        // pair is formed (pieces past K quantize zeros and are never stored)
        int q[NC][8];
        uint16_t dh[NC];
        float dmax = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (!CH && c * 2048 >= a.K) {  // uniform: whole chunks past K
#pragma unroll
                for (int i = 0; i < 8; ++i) q[c][i] = 0;
                dh[c] = 0;
                continue;
            }
            int qsum;
            quant8_block(v[c], q[c], dh[c], qsum);
            dmax = fmaxf(dmax, h2f(dh[c]));
        }
        dmax = xor_max<64>(dmax);
        if ((threadIdx.x & 63) == 0) redf[threadIdx.x >> 6] = dmax;
        __syncthreads();
        const float r = row_pow2(fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3])));
        if (threadIdx.x == 0) rs[m] = r;
        const float inv = 1.0f / r;  // exact: a power of two
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (!CH && c * 2048 >= a.K) break;
            const int t = c * 256 + (int)threadIdx.x;
            if ((t >> 2) >= nb) continue;
            uint4 hi, lo;
            split_dq8(q[c], dh[c], inv, hi, lo);
            uint16_t* row = y + m * y_stride + (int64_t)t * 8;
            *reinterpret_cast<uint4*>(row) = hi;
            *reinterpret_cast<uint4*>(row + a.K) = lo;
        }
    }
}

int act_prep_i8(const ActPrep& a, int64_t M, uint8_t* y, hipStream_t s) {
    if (M == 0) return GQ_OK;
    if (M > GEMM_I8_MAX_M || a.K > PREP_MAX_K || a.K % QK) return fail(GQ_ERR_UNSUPPORTED, "act_prep_i8: shape");
    const bool vec = ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0) && (a.xs % 4 == 0) &&
                     (!a.d || (((reinterpret_cast<uintptr_t>(a.d) & 15) == 0) && a.ds % 4 == 0)) &&
                     (reinterpret_cast<uintptr_t>(a.d2) & 15) == 0 && a.K % 4 == 0;
    uint16_t* yy = reinterpret_cast<uint16_t*>(y);
    const dim3 g((unsigned)M);
    // without RMS_NORM no value spans the row: one workgroup per row and 2048-element chunk
    // (measured at 8 rows, SWIGLU in front of the 7B down projection, K = 11008: 7.8 -> 4.8 us)
    if (!a.rms && a.K > 2048) {
        const dim3 gs((unsigned)M, (unsigned)cdiv(a.K, 2048));
        if (vec) hipLaunchKernelGGL((k_act_prep<true, 1, true, true>), gs, dim3(256), 0, s, a, yy, 0, nullptr);
        else hipLaunchKernelGGL((k_act_prep<false, 1, true, true>), gs, dim3(256), 0, s, a, yy, 0, nullptr);
        return check_hip(hipGetLastError(), "act_prep_i8 launch");
    }
    if (vec) {
        switch (cdiv(a.K, 2048)) {
            case 1: hipLaunchKernelGGL((k_act_prep<true, 1, true>), g, dim3(256), 0, s, a, yy, 0, nullptr); break;
            case 2: hipLaunchKernelGGL((k_act_prep<true, 2, true>), g, dim3(256), 0, s, a, yy, 0, nullptr); break;
            case 5: hipLaunchKernelGGL((k_act_prep<true, 5, true>), g, dim3(256), 0, s, a, yy, 0, nullptr); break;
            case 6: hipLaunchKernelGGL((k_act_prep<true, 6, true>), g, dim3(256), 0, s, a, yy, 0, nullptr); break;
            default: hipLaunchKernelGGL((k_act_prep<true, 0, true>), g, dim3(256), 0, s, a, yy, 0, nullptr); break;
        }
    } else {
        hipLaunchKernelGGL((k_act_prep<false, 0, true>), g, dim3(256), 0, s, a, yy, 0, nullptr);
    }
    return check_hip(hipGetLastError(), "act_prep_i8 launch");
}

int act_prep(const ActPrep& a, int64_t M, uint16_t* y, int64_t y_stride, float* rs, hipStream_t s) {
    if (M == 0) return GQ_OK;
    if (a.K > PREP_MAX_K || a.K % QK) return fail(GQ_ERR_UNSUPPORTED, "act_prep: K too large");
    const bool vec = ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0) && (a.xs % 4 == 0) &&
                     (!a.d || (((reinterpret_cast<uintptr_t>(a.d) & 15) == 0) && a.ds % 4 == 0)) &&
                     (reinterpret_cast<uintptr_t>(a.d2) & 15) == 0 && a.K % 4 == 0;
    const dim3 g((unsigned)M);
    if (vec) {  // the configs' K: 960 and 1536 (1 chunk), 2560 and 4096 (2), 8960 (5), 11008 (6)
        switch (cdiv(a.K, 2048)) {
            case 1: hipLaunchKernelGGL((k_act_prep<true, 1>), g, dim3(256), 0, s, a, y, y_stride, rs); break;
            case 2: hipLaunchKernelGGL((k_act_prep<true, 2>), g, dim3(256), 0, s, a, y, y_stride, rs); break;
            case 5: hipLaunchKernelGGL((k_act_prep<true, 5>), g, dim3(256), 0, s, a, y, y_stride, rs); break;
            case 6: hipLaunchKernelGGL((k_act_prep<true, 6>), g, dim3(256), 0, s, a, y, y_stride, rs); break;
            default: hipLaunchKernelGGL((k_act_prep<true, 0>), g, dim3(256), 0, s, a, y, y_stride, rs); break;
        }
    } else {
        hipLaunchKernelGGL((k_act_prep<false, 0>), g, dim3(256), 0, s, a, y, y_stride, rs);
    }
    return check_hip(hipGetLastError(), "act_prep launch");
}

// ---- weight quantizers (quantize.py semantics) ------------------------------

__global__ __launch_bounds__(256) void k_quant_w_q8_0(const float* __restrict__ x, uint8_t* __restrict__ y,
                                                      int64_t nblocks) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float* xb = x + b * QK;
    float v[QK];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < QK; ++j) {
        v[j] = xb[j];
        amax = fmaxf(amax, fabsf(v[j]));
    }
    const float scale = amax > 0.0f ? div_rn(amax, 127.0f) : 0.0f;
    const float inv = div_rn(1.0f, scale != 0.0f ? scale : 1.0f);
    uint8_t* o = y + b * Q8_BYTES;
    const uint16_t dh = f2h(scale);
    o[0] = (uint8_t)(dh & 0xff);
    o[1] = (uint8_t)(dh >> 8);
#pragma unroll
    for (int j = 0; j < QK; ++j) {
        float r = __builtin_rintf(v[j] * inv);
        r = fminf(fmaxf(r, -128.0f), 127.0f);
        o[2 + j] = (uint8_t)(int8_t)(int)r;
    }
}

__global__ __launch_bounds__(256) void k_quant_w_q4_0(const float* __restrict__ x, uint8_t* __restrict__ y,
                                                      int64_t nblocks) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float* xb = x + b * QK;
    float v[QK];
    float amax = -1.0f;
    float smax = 0.0f;
#pragma unroll
    for (int j = 0; j < QK; ++j) {
        v[j] = xb[j];
        const float a = fabsf(v[j]);
        if (a > amax) {  // first index of the largest magnitude (np.argmax)
            amax = a;
            smax = v[j];
        }
    }
    const float scale = smax != 0.0f ? smax / -8.0f : 0.0f;
    const float safe = scale != 0.0f ? scale : 1.0f;
    uint8_t q[QK];
#pragma unroll
    for (int j = 0; j < QK; ++j) {
        if (scale == 0.0f) {
            q[j] = 8;
        } else {
            float r = __builtin_rintf(div_rn(v[j], safe)) + 8.0f;
            r = fminf(fmaxf(r, 0.0f), 15.0f);
            q[j] = (uint8_t)(int)r;
        }
    }
    uint8_t* o = y + b * Q4_BYTES;
    const uint16_t dh = f2h(scale);
    o[0] = (uint8_t)(dh & 0xff);
    o[1] = (uint8_t)(dh >> 8);
#pragma unroll
    for (int j = 0; j < QK / 2; ++j) o[2 + j] = (uint8_t)((q[j] & 0x0f) | ((q[j + 16] & 0x0f) << 4));
}

int quantize_weights(int type, const float* x, void* y, int64_t n, hipStream_t s) {
    const int64_t nb = n / QK;
    if (nb == 0) return GQ_OK;
    const dim3 grid((unsigned)cdiv(nb, 256));
    if (type == GQ_TYPE_Q8_0)
        hipLaunchKernelGGL(k_quant_w_q8_0, grid, dim3(256), 0, s, x, (uint8_t*)y, nb);
    else
        hipLaunchKernelGGL(k_quant_w_q4_0, grid, dim3(256), 0, s, x, (uint8_t*)y, nb);
    return check_hip(hipGetLastError(), "quantize_weights launch");
}

}  // namespace gq
