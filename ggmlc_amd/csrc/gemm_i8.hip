// MUL_MAT for 5..16 activation rows (the batched decode of continuous batching) on int8
// MFMA (gfx950 v_mfma_i32_16x16x32_i8), for rows of K % 256 == 0.
//
// Semantics: ggml_mul_mat with src1 quantized to Q8_0 (quantize_row_q8_0): per quant
// block the exact integer sum isum = sum_j q_w[j] q_x[j], then acc += isum * (d_w * d_x)
// in fp32 (ggml-cpu/ggml-cpu.c:1164-1252; quants.c:225-256 Q4_0, :451-479 Q8_0). One
// MFMA yields isum for 16 weight rows x 16 activation rows of one block, exactly;
// d_w * d_x (two fp16 values) is exact in fp32, so each block adds one rounded product,
// as on the CPU. Q4_0 nibbles are dotted unsigned (0..15) and the block's 8 * sum(q_x)
// is subtracted, which keeps isum exact.
//
// Streaming: a wave owns 16 consecutive weight rows and walks a range of its K in steps
// of 8 blocks (272 B of a Q8_0 row, 144 B of a Q4_0 row: whole 16-byte chunks when
// K % 256 == 0). A step's 16 row segments are fetched with coalesced 16-byte raw buffer
// loads into a two-deep register ring, parked in the wave's LDS slice and read back as
// MFMA operands: lane l takes weight row l % 16 and quants 8 (l / 16) .. + 7 of a block
// (Q4_0: the low nibbles of bytes 8 ((l / 16) & 1) .. + 7, or their high nibbles for
// l / 16 >= 2). The activation operand (lane l: activation row l % 16, the same quants)
// and its scales and block sums come from the workspace written by the activation
// prologue (act_prep, i8 layout). D[i][j]: lane l holds activation row j = l % 16 and
// weight rows 4 (l / 16) .. + 3.
//
// K split: the 4 waves of a workgroup take 4 tiles (KS = 1), 2 tiles in 2 K parts or 1
// tile in 4 K parts; partial sums are added in part order through LDS, so results do
// not depend on timing.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace gq {

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int NBS = 8;  // quant blocks per step
constexpr uint32_t OOB = 0x80000000u;  // buffer offset past any resource: reads 0, no fetch

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int64_t bytes) {
    const uint64_t base = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
    const uint32_t n = bytes <= 0 ? 0u : (bytes > 0x7fffffff ? 0x7fffffffu : (uint32_t)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                             (int)__builtin_amdgcn_readfirstlane(n), 0x00020000);
}

template <int QT, int KS>
__global__ __launch_bounds__(256, 2) void k_gemm_i8(const uint8_t* __restrict__ W, int64_t N, int64_t K,
                                                    int64_t row_bytes, const uint8_t* __restrict__ act, int64_t M,
                                                    float* __restrict__ dst, int64_t ldd,
                                                    const float* __restrict__ bias) {
    constexpr int BB = QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES;
    constexpr int RB = NBS * BB;           // bytes of a row per step: 272 / 144
    constexpr int CPR = RB / 16;           // 16-byte chunks of a row per step: 17 / 9
    constexpr int CPW = 16 * CPR;          // chunks of a wave's step: 272 / 144
    constexpr int LPL = (CPW + 63) / 64;   // chunk loads per lane per step: 5 / 3
    __shared__ __align__(16) uint8_t s_stage[4][16 * RB];
    __shared__ float s_red[KS > 1 ? 4 : 1][64][4];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int g = lane >> 4, lr = lane & 15;
    const int64_t tile = (int64_t)blockIdx.x * (4 / KS) + wave / KS;
    const int kp = wave % KS;
    const int64_t n0 = tile * 16;
    const int nb = (int)(K / QK);
    const int nsteps = nb / NBS;
    const int sp = (nsteps + KS - 1) / KS;
    const int s0 = min(nsteps, kp * sp), s1 = min(nsteps, s0 + sp);

    // the tile's rows of W (rows past N, or a whole tile past N, read 0 without a fetch)
    const int64_t rows = N - n0;
    const __amdgpu_buffer_rsrc_t wrs =
        rsrc(W + (rows > 0 ? n0 : 0) * row_bytes, rows > 0 ? std::min<int64_t>(rows, 16) * row_bytes : 0);
    // activation workspace: quants [nb][16][32] int8, scales [nb][16] f32, block sums [nb][16] i32
    const __amdgpu_buffer_rsrc_t qrs = rsrc(act, (int64_t)nb * 512);
    const __amdgpu_buffer_rsrc_t drs = rsrc(act + (int64_t)nb * 512, (int64_t)nb * 64);
    const __amdgpu_buffer_rsrc_t srs = rsrc(act + (int64_t)nb * 576, (int64_t)nb * 64);

    // chunk i of a lane is chunk c = lane + 64 i of the step: row c / CPR, byte 16 (c % CPR)
    uint32_t coff[LPL];
    bool cval[LPL];
#pragma unroll
    for (int i = 0; i < LPL; ++i) {
        const int c = lane + 64 * i;
        cval[i] = c < CPW;
        coff[i] = cval[i] ? (uint32_t)((c / CPR) * row_bytes + (c % CPR) * 16) : 0u;
    }

    uint4 wb[2][LPL];
    u32x2 ab[2][NBS];
    float db[2][NBS];
    int sb[2][NBS];
    auto issue_w = [&](int s, int slot) {
        const bool live = s < s1;
#pragma unroll
        for (int i = 0; i < LPL; ++i) {
            const uint32_t off = live && cval[i] ? coff[i] + (uint32_t)s * RB : OOB;
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)off, 0, 0);
            wb[slot][i] = make_uint4(v.x, v.y, v.z, v.w);
        }
    };
    auto issue_a = [&](int s, int slot) {
        const bool live = s < s1;
#pragma unroll
        for (int b = 0; b < NBS; ++b) {
            const uint32_t e = (uint32_t)((s * NBS + b) * 16 + lr);  // (block, activation row)
            ab[slot][b] = __builtin_amdgcn_raw_buffer_load_b64(qrs, live ? (int)(e * 32 + 8 * g) : (int)OOB, 0, 0);
            db[slot][b] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(drs, live ? (int)(e * 4) : (int)OOB, 0, 0));
            if constexpr (QT == GQ_TYPE_Q4_0)
                sb[slot][b] = (int)__builtin_amdgcn_raw_buffer_load_b32(srs, live ? (int)(e * 4) : (int)OOB, 0, 0);
        }
    };

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    uint8_t* st = s_stage[wave];
    const int gq = QT == GQ_TYPE_Q8_0 ? g : (g & 1);  // the lane's 8 quant bytes of a block
    const int nsh = QT == GQ_TYPE_Q8_0 ? 0 : 4 * (g >> 1);  // Q4_0: low or high nibbles
    // one step from ring slot `slot`: park its weights, refill the slot with step s + 2,
    // then the 8 blocks' MFMAs
    auto body = [&](int s, int slot) {
#pragma unroll
        for (int i = 0; i < LPL; ++i)
            if (cval[i]) *reinterpret_cast<uint4*>(st + (lane + 64 * i) * 16) = wb[slot][i];
        wave_lds_sync();
        issue_w(s + 2, slot);
#pragma unroll
        for (int b = 0; b < NBS; ++b) {
            // weight operand: 8 bytes at row lr, block b, quant byte 8 gq (2 + 34 b / 18 b
            // from the segment start: 2 bytes off a dword boundary for even b)
            const uint8_t* rp = st + lr * RB + b * BB + 2 + 8 * gq;
            uint32_t lo, hi;
            if ((b & 1) == 0) {
                const uint32_t* p = reinterpret_cast<const uint32_t*>(rp - 2);
                const uint32_t d0 = p[0], d1 = p[1], d2 = p[2];
                lo = __builtin_amdgcn_alignbyte(d1, d0, 2);
                hi = __builtin_amdgcn_alignbyte(d2, d1, 2);
            } else {
                const uint32_t* p = reinterpret_cast<const uint32_t*>(rp);
                lo = p[0];
                hi = p[1];
            }
            if constexpr (QT == GQ_TYPE_Q4_0) {
                lo = (lo >> nsh) & 0x0f0f0f0fu;
                hi = (hi >> nsh) & 0x0f0f0f0fu;
            }
            const long wa = (long)(((uint64_t)hi << 32) | lo);
            const long xa = (long)(((uint64_t)ab[slot][b].y << 32) | ab[slot][b].x);
            const int4v zero = {0, 0, 0, 0};
            const int4v d = __builtin_amdgcn_mfma_i32_16x16x32_i8(wa, xa, zero, 0, 0, 0);
            const float dx = db[slot][b];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float dw = h2f(*reinterpret_cast<const uint16_t*>(st + (4 * g + r) * RB + b * BB));
                const int isum = QT == GQ_TYPE_Q8_0 ? d[r] : d[r] - 8 * sb[slot][b];
                acc[r] = __builtin_fmaf((float)isum, dw * dx, acc[r]);
            }
        }
        wave_lds_sync();  // the slice is read before the next step parks
        issue_a(s + 2, slot);
    };

    issue_w(s0, 0);
    issue_a(s0, 0);
    issue_w(s0 + 1, 1);
    issue_a(s0 + 1, 1);
    int s = s0;
    for (; s + 1 < s1; s += 2) {
        body(s, 0);
        body(s + 1, 1);
    }
    if (s < s1) body(s, 0);

    if constexpr (KS > 1) {
#pragma unroll
        for (int r = 0; r < 4; ++r) s_red[wave][lane][r] = acc[r];
        __syncthreads();
        if (kp != 0) return;
#pragma unroll
        for (int k = 1; k < KS; ++k)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] += s_red[wave + k][lane][r];
    }
    const int64_t m = lr;  // activation row
    if (m >= M) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t n = n0 + 4 * g + r;
        if (n < N) dst[m * ldd + n] = bias ? acc[r] + bias[n] : acc[r];
    }
}

template <int QT>
int launch(const uint8_t* W, int64_t N, int64_t K, const uint8_t* act, int64_t M, float* dst, int64_t ldd,
           hipStream_t s, const float* bias) {
    const int64_t row_bytes = (K / QK) * (QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES);
    const GemmI8Plan p = gemm_i8_plan(N, K);
    const dim3 grid((unsigned)p.wgs);
    if (p.ks == 4)
        hipLaunchKernelGGL((k_gemm_i8<QT, 4>), grid, dim3(256), 0, s, W, N, K, row_bytes, act, M, dst, ldd, bias);
    else if (p.ks == 2)
        hipLaunchKernelGGL((k_gemm_i8<QT, 2>), grid, dim3(256), 0, s, W, N, K, row_bytes, act, M, dst, ldd, bias);
    else
        hipLaunchKernelGGL((k_gemm_i8<QT, 1>), grid, dim3(256), 0, s, W, N, K, row_bytes, act, M, dst, ldd, bias);
    return check_hip(hipGetLastError(), "gemm_i8 launch");
}

}  // namespace

// K parts per 16-row tile, for rows of at least 4 steps: 4 below 512 tiles, 2 below 4096
// (measured at M = 16: Qwen2.5-1.5B qkv 7.9 -> 7.2 us, gate_up 18.5 -> 16.4 us, 7B
// gate_up 38.5 -> 32.7 us against one part; the 152k-row head keeps one)
GemmI8Plan gemm_i8_plan(int64_t N, int64_t K) {
    GemmI8Plan p;
    const int64_t tiles = cdiv(N, 16), nsteps = K / (QK * NBS);
    p.ks = 1;
    if (tiles < 512 && nsteps >= 4) p.ks = 4;
    else if (tiles < 4096 && nsteps >= 4) p.ks = 2;
    p.wgs = cdiv(tiles, 4 / p.ks);
    return p;
}

int gemm_i8(int type, const uint8_t* W, int64_t N, int64_t K, const uint8_t* act, int64_t M, float* dst,
            int64_t ldd, hipStream_t s, const float* bias) {
    if (K % GEMM_I8_K_ALIGN != 0 || M < 1 || M > GEMM_I8_MAX_M)
        return fail(GQ_ERR_INVALID, "gemm_i8: needs K % 256 == 0 and 1 <= M <= 16");
    if ((reinterpret_cast<uintptr_t>(W) & 15) != 0 || (reinterpret_cast<uintptr_t>(act) & 15) != 0)
        return fail(GQ_ERR_INVALID, "gemm_i8: weight and activation must be 16-byte aligned");
    if (type == GQ_TYPE_Q8_0) return launch<GQ_TYPE_Q8_0>(W, N, K, act, M, dst, ldd, s, bias);
    return launch<GQ_TYPE_Q4_0>(W, N, K, act, M, dst, ldd, s, bias);
}

}  // namespace gq
