// Decode GEMV over native ggml Q8_0 / Q4_0 rows (dst[m, n] = W[n, :] . x[m, :]).
//
// Semantics: ggml_compute_forward_mul_mat's vec_dot path for src1 quantized to
// Q8_0 (ggml-cpu/ggml-cpu.c:1164-1252; per-block integer dot, then
// d_w * d_x * isum accumulated: ggml-cpu/quants.c:225-256 Q4_0, :451-479 Q8_0).
//
// Streaming design (K % 256 == 0, every config of the north star except K = 960):
// a row of K elements is K/256 "groups" of 8 blocks; a group is 272 B (Q8_0) or
// 144 B (Q4_0), a whole number of 16-byte chunks. Each wave owns 4 rows; per
// iteration it streams 16 consecutive groups of each row with coalesced 16-byte
// loads (every wave instruction reads 1 KiB of contiguous weight bytes), parks
// them in its private LDS slice, and each lane then pulls back one whole group
// (17 or 9 aligned ds_read_b128) and decodes the 8 blocks in registers: the fp16
// scale sits at byte 34b (18b) and the quants start 2 bytes later, so blocks
// with an even index are realigned with v_alignbyte and odd ones are already
// dword aligned. Integer dots use v_dot4_i32_i8; Q4_0 nibbles are dotted
// unsigned and corrected with the precomputed block sum of the activation
// (isum = dot(n, a) - 8 * sum(a)), which keeps the block sum exact.
// The next iteration's global loads are issued before the current group is
// decoded (register double buffer). The quantized activation (ACT_GS layout,
// written by the quantizer) is copied to LDS once per workgroup.
// A 16-lane xor reduction finishes each row.
//
// Fallback (any K % 32 == 0): one lane per block with 16-bit loads.
#include "common.h"
#include "kernels.h"

namespace gq {

namespace {

constexpr int LPR = 16;        // lanes per row (consecutive groups of one row)
constexpr int RPW = 64 / LPR;  // rows per wave
constexpr int WAVES = 4;

template <int QT>
struct QTraits;
template <>
struct QTraits<GQ_TYPE_Q8_0> {
    static constexpr int BB = Q8_BYTES;
    static constexpr int GB = 8 * BB;   // 272
    static constexpr int CPG = GB / 16; // 17
    static constexpr int NQW = 8;       // quant dwords per block
};
template <>
struct QTraits<GQ_TYPE_Q4_0> {
    static constexpr int BB = Q4_BYTES;
    static constexpr int GB = 8 * BB;   // 144
    static constexpr int CPG = GB / 16; // 9
    static constexpr int NQW = 4;
};

template <int QT>
__device__ __forceinline__ void decode_block(const uint32_t* w, int b, uint32_t& hdr, uint32_t* q) {
    constexpr int BB = QTraits<QT>::BB;
    constexpr int NQW = QT == GQ_TYPE_Q8_0 ? 8 : 4;  // quant dwords per block
    constexpr int DWB = BB / 2;                      // dwords per 2 blocks (17 / 9)
    if ((b & 1) == 0) {
        const int base = (b / 2) * DWB;
        hdr = w[base] & 0xffffu;
#pragma unroll
        for (int i = 0; i < NQW; ++i) q[i] = __builtin_amdgcn_alignbyte(w[base + i + 1], w[base + i], 2);
    } else {
        const int base = (b / 2) * DWB + DWB / 2;  // (BB*b - 2)/4
        hdr = w[base] >> 16;
#pragma unroll
        for (int i = 0; i < NQW; ++i) q[i] = w[base + 1 + i];
    }
}

// integer dot of one weight block (decoded quant dwords q) with the activation
// block (a0, a1 = its 32 int8); Q4_0 nibbles are biased by 8 via the block sum
template <int QT>
__device__ __forceinline__ int block_dot(const uint32_t* q, const uint4& a0, const uint4& a1,
                                         const uint8_t* ag, int bi) {
    if constexpr (QT == GQ_TYPE_Q8_0) {
        int s = dot4(q[0], a0.x, 0);
        s = dot4(q[1], a0.y, s);
        s = dot4(q[2], a0.z, s);
        s = dot4(q[3], a0.w, s);
        s = dot4(q[4], a1.x, s);
        s = dot4(q[5], a1.y, s);
        s = dot4(q[6], a1.z, s);
        return dot4(q[7], a1.w, s);
    } else {
        const int sa = reinterpret_cast<const int*>(ag + ACT_S_OFF)[bi];
        int s = dot4(q[0] & 0x0f0f0f0fu, a0.x, -8 * sa);
        s = dot4(q[1] & 0x0f0f0f0fu, a0.y, s);
        s = dot4(q[2] & 0x0f0f0f0fu, a0.z, s);
        s = dot4(q[3] & 0x0f0f0f0fu, a0.w, s);
        s = dot4((q[0] >> 4) & 0x0f0f0f0fu, a1.x, s);
        s = dot4((q[1] >> 4) & 0x0f0f0f0fu, a1.y, s);
        s = dot4((q[2] >> 4) & 0x0f0f0f0fu, a1.z, s);
        return dot4((q[3] >> 4) & 0x0f0f0f0fu, a1.w, s);
    }
}

template <int QT, int M>
__global__ __launch_bounds__(256, 2) void k_gemv_grp(const uint8_t* __restrict__ W, int64_t N,
                                                     int64_t row_bytes, int G,
                                                     const uint8_t* __restrict__ act,
                                                     int64_t act_stride, float* __restrict__ dst,
                                                     int64_t ldd) {
    constexpr int GB = QTraits<QT>::GB;
    constexpr int CPG = QTraits<QT>::CPG;
    constexpr int SEG = LPR * CPG;  // chunks of one row per iteration
    extern __shared__ __align__(16) uint8_t smem[];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int act_bytes = G * ACT_GS;
    uint8_t* s_act = smem;
    uint8_t* s_stage = smem + M * act_bytes + wave * 64 * GB;

    // activation rows -> LDS (whole ACT_GS groups, 16-byte copies)
    for (int m = 0; m < M; ++m)
        for (int off = threadIdx.x * 16; off < act_bytes; off += 256 * 16)
            *reinterpret_cast<uint4*>(s_act + m * act_bytes + off) =
                *reinterpret_cast<const uint4*>(act + m * act_stride + off);

    const int64_t row0 = ((int64_t)blockIdx.x * WAVES + wave) * RPW;
    const int rsub = lane / LPR;
    const int gsub = lane % LPR;
    const int64_t row = row0 + rsub;
    const int J = (G + LPR - 1) / LPR;

    uint4 pre[CPG];
    auto load_iter = [&](int j) {
#pragma unroll
        for (int c = 0; c < CPG; ++c) {
            const int ci = lane + 64 * c;
            const int r = ci / SEG;
            const int within = ci - r * SEG;
            const int64_t rr = row0 + r;
            const int64_t boff = (int64_t)j * (LPR * GB) + (int64_t)within * 16;
            if (rr < N && boff < row_bytes)
                pre[c] = ld_nt16(W + rr * row_bytes + boff);
            else
                pre[c] = make_uint4(0, 0, 0, 0);
        }
    };

    load_iter(0);
    __syncthreads();  // activation in LDS

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;

    for (int j = 0; j < J; ++j) {
#pragma unroll
        for (int c = 0; c < CPG; ++c) *reinterpret_cast<uint4*>(s_stage + (lane + 64 * c) * 16) = pre[c];
        wave_lds_sync();
        if (j + 1 < J) load_iter(j + 1);
        uint32_t w[4 * CPG];
#pragma unroll
        for (int c = 0; c < CPG; ++c) {
            const uint4 t = *reinterpret_cast<const uint4*>(s_stage + lane * GB + 16 * c);
            w[4 * c + 0] = t.x;
            w[4 * c + 1] = t.y;
            w[4 * c + 2] = t.z;
            w[4 * c + 3] = t.w;
        }
        wave_lds_sync();
        const int g = j * LPR + gsub;
        if (row < N && g < G) {
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                uint32_t hdr;
                uint32_t q[QTraits<QT>::NQW];
                decode_block<QT>(w, b, hdr, q);
                const float dw = h2f((uint16_t)hdr);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const uint8_t* ag = s_act + m * act_bytes + g * ACT_GS;
                    const uint4 a0 = *reinterpret_cast<const uint4*>(ag + ACT_QS_OFF + 32 * b);
                    const uint4 a1 = *reinterpret_cast<const uint4*>(ag + ACT_QS_OFF + 32 * b + 16);
                    const float da = reinterpret_cast<const float*>(ag + ACT_D_OFF)[b];
                    const int s = block_dot<QT>(q, a0, a1, ag, b);
                    acc[m] += (float)s * (dw * da);
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float v = xor_sum<LPR>(acc[m]);
        if (gsub == 0 && row < N) dst[(int64_t)m * ldd + row] = v;
    }
}

// ---- fallback: one lane per block, 16-bit loads (any K % 32 == 0) ---------------

template <int QT, int M>
__global__ __launch_bounds__(256) void k_gemv_blk(const uint8_t* __restrict__ W, int64_t N,
                                                  int64_t row_bytes, int nb,
                                                  const uint8_t* __restrict__ act,
                                                  int64_t act_stride, float* __restrict__ dst,
                                                  int64_t ldd) {
    constexpr int BB = QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES;
    constexpr int NQW = QT == GQ_TYPE_Q8_0 ? 8 : 4;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
    const int sub = lane % LPR;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;
    if (row < N) {
        const uint8_t* rp = W + row * row_bytes;
        for (int b = sub; b < nb; b += LPR) {
            const uint16_t* bp = reinterpret_cast<const uint16_t*>(rp + (int64_t)b * BB);
            const float dw = h2f(bp[0]);
            uint32_t q[NQW];
#pragma unroll
            for (int i = 0; i < NQW; ++i) q[i] = (uint32_t)bp[1 + 2 * i] | ((uint32_t)bp[2 + 2 * i] << 16);
            const int g = b >> 3, bi = b & 7;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint8_t* ag = act + m * act_stride + (int64_t)g * ACT_GS;
                const uint4 a0 = *reinterpret_cast<const uint4*>(ag + ACT_QS_OFF + 32 * bi);
                const uint4 a1 = *reinterpret_cast<const uint4*>(ag + ACT_QS_OFF + 32 * bi + 16);
                const float da = reinterpret_cast<const float*>(ag + ACT_D_OFF)[bi];
                const int s = block_dot<QT>(q, a0, a1, ag, bi);
                acc[m] += (float)s * (dw * da);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float v = xor_sum<LPR>(acc[m]);
        if (sub == 0 && row < N) dst[(int64_t)m * ldd + row] = v;
    }
}

template <int QT, int M>
int launch_grp(const uint8_t* W, int64_t N, int64_t K, const uint8_t* act, int64_t act_stride,
               float* dst, int64_t ldd, hipStream_t s) {
    const int G = (int)(K / 256);
    const int64_t row_bytes = (K / QK) * QTraits<QT>::BB;
    const size_t lds = (size_t)M * G * ACT_GS + (size_t)WAVES * 64 * QTraits<QT>::GB;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv_grp<QT, M>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return check_hip(e, "gemv set LDS attribute");
        attr_set = true;
    }
    if (lds > 160 * 1024) return fail(GQ_ERR_UNSUPPORTED, "gemv: activation too large for LDS");
    const dim3 grid((unsigned)cdiv(N, WAVES * RPW));
    hipLaunchKernelGGL((k_gemv_grp<QT, M>), grid, dim3(256), lds, s, W, N, row_bytes, G, act,
                       act_stride, dst, ldd);
    return check_hip(hipGetLastError(), "gemv launch");
}

template <int QT, int M>
int launch_blk(const uint8_t* W, int64_t N, int64_t K, const uint8_t* act, int64_t act_stride,
               float* dst, int64_t ldd, hipStream_t s) {
    const int nb = (int)(K / QK);
    const int64_t row_bytes = (int64_t)nb * (QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES);
    const dim3 grid((unsigned)cdiv(N, 256 / LPR));
    hipLaunchKernelGGL((k_gemv_blk<QT, M>), grid, dim3(256), 0, s, W, N, row_bytes, nb, act,
                       act_stride, dst, ldd);
    return check_hip(hipGetLastError(), "gemv launch");
}

template <int QT>
int gemv_t(const uint8_t* W, int64_t N, int64_t K, const uint8_t* act, int64_t act_stride, int64_t M,
           float* dst, int64_t ldd, hipStream_t s) {
    const bool grp = (K % 256 == 0) && ((reinterpret_cast<uintptr_t>(W) & 15) == 0);
    switch (M) {
        case 1: return grp ? launch_grp<QT, 1>(W, N, K, act, act_stride, dst, ldd, s)
                           : launch_blk<QT, 1>(W, N, K, act, act_stride, dst, ldd, s);
        case 2: return grp ? launch_grp<QT, 2>(W, N, K, act, act_stride, dst, ldd, s)
                           : launch_blk<QT, 2>(W, N, K, act, act_stride, dst, ldd, s);
        case 3: return grp ? launch_grp<QT, 3>(W, N, K, act, act_stride, dst, ldd, s)
                           : launch_blk<QT, 3>(W, N, K, act, act_stride, dst, ldd, s);
        case 4: return grp ? launch_grp<QT, 4>(W, N, K, act, act_stride, dst, ldd, s)
                           : launch_blk<QT, 4>(W, N, K, act, act_stride, dst, ldd, s);
        default: return fail(GQ_ERR_INVALID, "gemv: M out of range");
    }
}

}  // namespace

int gemv(int type, const uint8_t* W, int64_t N, int64_t K, const uint8_t* act, int64_t act_stride,
         int64_t M, float* dst, int64_t ldd, hipStream_t s) {
    if (type == GQ_TYPE_Q8_0) return gemv_t<GQ_TYPE_Q8_0>(W, N, K, act, act_stride, M, dst, ldd, s);
    return gemv_t<GQ_TYPE_Q4_0>(W, N, K, act, act_stride, M, dst, ldd, s);
}

}  // namespace gq
