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
// decoded (register double buffer). Each workgroup first quantizes the fp32
// activation rows into LDS itself (ACT_GS layout, the exact rule of
// quantize_row_q8_0), so a decode MUL_MAT is a single launch.
// A 16-lane xor reduction finishes each row.
//
// Fallback (any K % 32 == 0): one lane per block with 16-bit loads, activation
// quantized into LDS the same way.
#include <mutex>
#include <unordered_map>

#include "common.h"
#include "kernels.h"

#pragma clang fp contract(off)

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
    static constexpr int HC = 9;        // 16-byte chunks of a half-group window
    static constexpr int H1 = 8;        // first chunk of the second window (byte 128)
};
template <>
struct QTraits<GQ_TYPE_Q4_0> {
    static constexpr int BB = Q4_BYTES;
    static constexpr int GB = 8 * BB;   // 144
    static constexpr int CPG = GB / 16; // 9
    static constexpr int NQW = 4;
    static constexpr int HC = 5;        // windows: bytes [0, 80) and [64, 144)
    static constexpr int H1 = 4;
};

// Block at byte offset o (even) of a dword window w: its fp16 scale and quant
// dwords. o % 4 == 0 puts the scale in the low half of w[o/4] and the quants two
// bytes later (realigned with v_alignbyte); o % 4 == 2 puts the scale in the
// high half and the quants on a dword boundary.
template <int QT>
__device__ __forceinline__ void decode_at(const uint32_t* w, int o, uint32_t& hdr, uint32_t* q) {
    constexpr int NQW = QTraits<QT>::NQW;
    if ((o & 3) == 0) {
        const int base = o >> 2;
        hdr = w[base] & 0xffffu;
#pragma unroll
        for (int i = 0; i < NQW; ++i) q[i] = __builtin_amdgcn_alignbyte(w[base + i + 1], w[base + i], 2);
    } else {
        const int base = (o - 2) >> 2;
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

// Physical weight row of logical row r: with the SWIGLU epilogue, logical rows
// 2c and 2c+1 are the gate row c and the up row c + N/2, so both land in the same
// wave (rows of a wave are 4 consecutive logical rows).
__device__ __forceinline__ int64_t phys_row(const GemvFuse& fz, int64_t r) {
    return fz.glu ? (r >> 1) + (r & 1) * fz.glu_half : r;
}

// silu(g) * u with the arithmetic of k_swiglu (x / (1 + expf(-x)) * g)
__device__ __forceinline__ float swiglu1(float g, float u) {
    const float sg = g / (1.0f + expf(-g));
    return sg * u;
}

// Write logical row `row` of activation m: plain, residual-added (res + v: the
// operand order of ADD(x, MUL_MAT)), or, for the SWIGLU epilogue, from the even
// row with its partner's value vp.
__device__ __forceinline__ void emit(const GemvFuse& fz, float* dst, int64_t ldd, int m, int64_t row, float v,
                                     float vp) {
    if (fz.glu) {
        if ((row & 1) == 0) dst[(int64_t)m * ldd + (row >> 1)] = swiglu1(v, vp);
        return;
    }
    if (fz.res) v = fz.res[(int64_t)m * fz.ldr + row] + v;
    dst[(int64_t)m * ldd + row] = v;
}

template <int QT, int M, bool XVEC, int PF, int KS>
__global__ __launch_bounds__(256, 2) void k_gemv_grp(const uint8_t* __restrict__ W, int64_t N,
                                                     int64_t row_bytes, int G,
                                                     const float* __restrict__ x,
                                                     int64_t x_stride, float* dst,
                                                     int64_t ldd, GemvFuse fz) {
    constexpr int GB = QTraits<QT>::GB;
    constexpr int CPG = QTraits<QT>::CPG;
    constexpr int SEG = LPR * CPG;       // chunks of one row per step
    constexpr int XPMAX = 2;             // activation passes held in registers
    constexpr int RG = WAVES / KS;       // row groups (of RPW rows) per workgroup tile
    constexpr int ROWS = RG * RPW;       // rows per workgroup tile
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float red[WAVES][M][RPW];
    __shared__ double red_d[4];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int act_bytes = G * ACT_GS;
    uint8_t* s_act = smem;
    uint8_t* s_stage = smem + M * act_bytes + wave * 64 * GB;

    const int rsub = lane / LPR;
    const int gsub = lane % LPR;
    const int nb = G * 8;
    const int XP = (nb * 4 + 255) / 256;

    // wave -> (row group, K part); K parts are whole steps of LPR groups so every
    // step stays a full 64-group slice (a part may be empty: it then runs one
    // masked step so that all waves meet the same reduction barriers)
    const int rg = wave / KS;
    const int kp = wave % KS;
    const int J = (G + LPR - 1) / LPR;
    const int SP = (J + KS - 1) / KS;  // steps per part
    const int g_begin = min(G, kp * SP * LPR);
    const int g_end = min(G, (kp + 1) * SP * LPR);
    const int S = max(1, (g_end - g_begin + LPR - 1) / LPR);  // steps per tile for this wave

    // persistent workgroups over workgroup tiles; one flat (tile, step) pipeline per wave
    const int64_t n_wgt = (N + ROWS - 1) / ROWS;
    const int64_t my_wgt = blockIdx.x < n_wgt ? (n_wgt - blockIdx.x + gridDim.x - 1) / gridDim.x : 0;
    const int64_t F = my_wgt * S;

    float xr[XPMAX][8];
    const bool xpre = M * XP <= XPMAX;
    if (xpre) {
#pragma unroll
        for (int p = 0; p < XPMAX; ++p) {
            if (p < M * XP) {
                const int m = p / XP, t = (p - m * XP) * 256 + (int)threadIdx.x;
                load8<XVEC>(x + (int64_t)m * x_stride + (int64_t)(t >> 2) * QK + (t & 3) * 8, (t >> 2) < nb, xr[p]);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    uint4 pre[PF][CPG];
    auto load_step = [&](int64_t f, uint4(&dstv)[CPG]) {
        const int64_t t = (int64_t)blockIdx.x + (f / S) * gridDim.x;
        const int j = (int)(f % S);
        const int64_t row0 = t * ROWS + rg * RPW;
        const int gfirst = g_begin + j * LPR;             // first group of this step
        const int ngr = min(LPR, g_end - gfirst);          // groups of this step
#pragma unroll
        for (int c = 0; c < CPG; ++c) {
            const int ci = lane + 64 * c;
            const int r = ci / SEG;
            const int within = ci - r * SEG;
            const int64_t rr = row0 + r;
            const bool ok = rr < N && within < ngr * CPG;
            const int64_t boff = (int64_t)gfirst * GB + (int64_t)within * 16;
            // always-valid address, zeroed after the load: no branch per chunk
            uint4 v = ld_nt16(W + (ok ? phys_row(fz, rr) * row_bytes + boff : 0));
            if (!ok) v = make_uint4(0, 0, 0, 0);
            dstv[c] = v;
        }
    };
#pragma unroll
    for (int s = 0; s < PF; ++s)
        if (s < F) load_step(s, pre[s]);
    __builtin_amdgcn_sched_barrier(0);

    float scale[M];
#pragma unroll
    for (int m = 0; m < M; ++m) scale[m] = 1.0f;
    if (xpre) {
        if (fz.rms) {  // RMS_NORM fused: the rows' squares are already in registers
#pragma unroll
            for (int m = 0; m < M; ++m) {
                double sq = 0.0;
#pragma unroll
                for (int p = 0; p < XPMAX; ++p)
                    if (p < M * XP && p / XP == m) sq = sumsq8(xr[p], sq);
                scale[m] = rms_scale(block_sum_d(sq, red_d), (int64_t)G * 256, fz.eps);
            }
        }
#pragma unroll
        for (int p = 0; p < XPMAX; ++p) {
            if (p < M * XP) {  // uniform across the workgroup
                const int m = p / XP, t = (p - m * XP) * 256 + (int)threadIdx.x;
                const int b = t >> 2, part = t & 3;
#pragma unroll
                for (int i = 0; i < 8; ++i) xr[p][i] = xr[p][i] * scale[m];
                int q[8];
                uint16_t dh;
                int qsum;
                quant8_block(xr[p], q, dh, qsum);
                if (b < nb) {
                    uint8_t* gp = s_act + m * act_bytes + (b >> 3) * ACT_GS;
                    const int bi = b & 7;
                    uint32_t lo = 0, hi = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        lo |= (uint32_t)(q[i] & 0xff) << (8 * i);
                        hi |= (uint32_t)(q[4 + i] & 0xff) << (8 * i);
                    }
                    *reinterpret_cast<uint2*>(gp + ACT_QS_OFF + bi * QK + part * 8) = make_uint2(lo, hi);
                    if (part == 0) {
                        reinterpret_cast<float*>(gp + ACT_D_OFF)[bi] = h2f(dh);
                        reinterpret_cast<int*>(gp + ACT_S_OFF)[bi] = qsum;
                    }
                }
            }
        }
    } else {
        if (fz.rms) rms_scales<XVEC, M>(x, x_stride, M, G * 256, fz.eps, scale, red_d);
        quantize_rows_to_act<XVEC, M>(x, x_stride, M, G * 256, s_act, act_bytes, scale);
    }
    __syncthreads();  // quantized activation visible to all waves

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;

    for (int64_t f = 0; f < F; ++f) {
        const int64_t t = (int64_t)blockIdx.x + (f / S) * gridDim.x;
        const int j = (int)(f % S);
        const int64_t row = t * ROWS + rg * RPW + rsub;
#pragma unroll
        for (int c = 0; c < CPG; ++c) *reinterpret_cast<uint4*>(s_stage + (lane + 64 * c) * 16) = pre[0][c];
        wave_lds_sync();
        // rotate the register pipeline and issue step f + PF
#pragma unroll
        for (int s = 0; s + 1 < PF; ++s)
#pragma unroll
            for (int c = 0; c < CPG; ++c) pre[s][c] = pre[s + 1][c];
        if (f + PF < F) load_step(f + PF, pre[PF - 1]);
        const int g = g_begin + j * LPR + gsub;
        const bool live = row < N && g < g_end;
        // decode the group in two windows of HC chunks (blocks 0-3, then 4-7)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            constexpr int HC = QTraits<QT>::HC;
            const int c0 = h ? QTraits<QT>::H1 : 0;
            uint32_t w[4 * HC];
#pragma unroll
            for (int c = 0; c < HC; ++c) {
                const uint4 tt = *reinterpret_cast<const uint4*>(s_stage + gsub * GB + rsub * (LPR * GB) + 16 * (c0 + c));
                w[4 * c + 0] = tt.x;
                w[4 * c + 1] = tt.y;
                w[4 * c + 2] = tt.z;
                w[4 * c + 3] = tt.w;
            }
            if (!live) continue;
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
                const int b = 4 * h + bb;
                uint32_t hdr;
                uint32_t q[QTraits<QT>::NQW];
                decode_at<QT>(w, QTraits<QT>::BB * b - 16 * c0, hdr, q);
                const float dw = h2f((uint16_t)hdr);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const uint8_t* ag = s_act + m * act_bytes + g * ACT_GS;
                    const uint4 a0 = *reinterpret_cast<const uint4*>(ag + ACT_QS_OFF + 32 * b);
                    const uint4 a1 = *reinterpret_cast<const uint4*>(ag + ACT_QS_OFF + 32 * b + 16);
                    const float da = reinterpret_cast<const float*>(ag + ACT_D_OFF)[b];
                    const int sdot = block_dot<QT>(q, a0, a1, ag, b);
                    acc[m] += (float)sdot * (dw * da);
                }
            }
        }
        wave_lds_sync();  // this step's staging slice is fully read before it is refilled
        if (j == S - 1) {  // tile finished: reduce the 16 lanes of each row, then the K parts
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float v = xor_sum<LPR>(acc[m]);
                acc[m] = 0.0f;
                if constexpr (KS == 1) {
                    const float vp = __shfl_xor(v, LPR, 64);  // the next row's value (SWIGLU pairs)
                    if (gsub == 0 && row < N) emit(fz, dst, ldd, m, row, v, vp);
                } else {
                    if (gsub == 0) red[wave][m][rsub] = v;
                }
            }
            if constexpr (KS > 1) {
                __syncthreads();
                if (kp == 0 && gsub == 0 && row < N) {
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        float v = red[wave][m][rsub], vp = red[wave][m][rsub ^ 1];
#pragma unroll
                        for (int k = 1; k < KS; ++k) v += red[wave + k][m][rsub], vp += red[wave + k][m][rsub ^ 1];
                        emit(fz, dst, ldd, m, row, v, vp);
                    }
                }
                __syncthreads();
            }
        }
    }
}

// ---- fallback: one lane per block, 16-bit loads (any K % 32 == 0) ---------------

template <int QT, int M, bool XVEC>
__global__ __launch_bounds__(256) void k_gemv_blk(const uint8_t* __restrict__ W, int64_t N,
                                                  int64_t row_bytes, int nb,
                                                  const float* __restrict__ x,
                                                  int64_t x_stride, float* dst,
                                                  int64_t ldd, GemvFuse fz) {
    constexpr int BB = QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES;
    constexpr int NQW = QT == GQ_TYPE_Q8_0 ? 8 : 4;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red_d[4];
    const int act_stride = (int)act_row_bytes((int64_t)nb * QK);
    const uint8_t* act = smem;
    float scale[M];
#pragma unroll
    for (int m = 0; m < M; ++m) scale[m] = 1.0f;
    if (fz.rms) rms_scales<XVEC, M>(x, x_stride, M, nb * QK, fz.eps, scale, red_d);
    quantize_rows_to_act<XVEC, M>(x, x_stride, M, nb * QK, smem, act_stride, scale);
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
    const int sub = lane % LPR;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;
    if (row < N) {
        const uint8_t* rp = W + phys_row(fz, row) * row_bytes;
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
        const float vp = __shfl_xor(v, LPR, 64);
        if (sub == 0 && row < N) emit(fz, dst, ldd, m, row, v, vp);
    }
}

constexpr size_t LDS_MAX = 160 * 1024;

// dynamic LDS above 64 KiB must be allowed per kernel; `allowed` remembers the
// largest size granted so far (the attribute excludes the kernel's static LDS)
template <typename KFn>
int allow_big_lds(KFn* fn, size_t& allowed, size_t need) {
    if (need <= allowed || need <= 64 * 1024) return GQ_OK;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)need);
    if (e != hipSuccess) return check_hip(e, "gemv: set LDS attribute");
    allowed = need;
    return GQ_OK;
}

// persistent grid: as many workgroups as can be resident, never more than
// tiles (residency depends on the kernel and its LDS size: cached per pair)
template <typename KFn>
int resident_wgs(KFn* fn, size_t lds, int& out) {
    static std::mutex mu;
    static std::unordered_map<size_t, int> cache;
    const size_t key = lds * 1315423911u ^ reinterpret_cast<uintptr_t>(fn);
    {
        std::lock_guard<std::mutex> lk(mu);
        auto it = cache.find(key);
        if (it != cache.end()) {
            out = it->second;
            return GQ_OK;
        }
    }
    int per_cu = 0, ncu = 0, dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    rc = check_hip(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev), "CU count");
    if (rc) return rc;
    rc = check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, lds), "gemv occupancy");
    if (rc) return rc;
    out = (per_cu > 0 ? per_cu : 1) * ncu;
    std::lock_guard<std::mutex> lk(mu);
    cache[key] = out;
    return GQ_OK;
}

template <int QT, int M, bool XVEC, int PF, int KS>
int launch_grp_ks(const uint8_t* W, int64_t N, int64_t K, const float* x, int64_t x_stride,
                  float* dst, int64_t ldd, const GemvFuse& fz, hipStream_t s, size_t lds, int resident) {
    const int G = (int)(K / 256);
    const int64_t row_bytes = (K / QK) * QTraits<QT>::BB;
    auto* fn = &k_gemv_grp<QT, M, XVEC, PF, KS>;
    static size_t allowed = 0;
    int rc = allow_big_lds(fn, allowed, lds);
    if (rc) return rc;
    const int64_t tiles = cdiv(N, (WAVES / KS) * RPW);
    const dim3 grid((unsigned)(tiles < resident ? tiles : resident));
    hipLaunchKernelGGL(fn, grid, dim3(256), lds, s, W, N, row_bytes, G, x, x_stride, dst, ldd, fz);
    return check_hip(hipGetLastError(), "gemv launch");
}

template <int QT, int M, bool XVEC, int PF>
int launch_grp_pf(const uint8_t* W, int64_t N, int64_t K, const float* x, int64_t x_stride,
                  float* dst, int64_t ldd, const GemvFuse& fz, hipStream_t s) {
    const int G = (int)(K / 256);
    const size_t lds = (size_t)M * G * ACT_GS + (size_t)WAVES * 64 * QTraits<QT>::GB;
    if (lds > LDS_MAX) return fail(GQ_ERR_UNSUPPORTED, "gemv: activation too large for LDS");
    // residency is the same for every KS (same registers and LDS)
    int resident = 0;
    int rc = resident_wgs(&k_gemv_grp<QT, M, XVEC, PF, 1>, lds, resident);
    if (rc) return rc;
    // split K over the waves of a workgroup (whole steps per wave) only when
    // the row tiles leave most CUs without a workgroup (measured: splitting a
    // 4096-row down projection is slower, a 1536-row one faster)
    const int64_t t1 = cdiv(N, WAVES * RPW);
    const int J = (G + LPR - 1) / LPR;
    if (4 * t1 >= resident || J < 2)
        return launch_grp_ks<QT, M, XVEC, PF, 1>(W, N, K, x, x_stride, dst, ldd, fz, s, lds, resident);
    if (J < 3) return launch_grp_ks<QT, M, XVEC, PF, 2>(W, N, K, x, x_stride, dst, ldd, fz, s, lds, resident);
    return launch_grp_ks<QT, M, XVEC, PF, 4>(W, N, K, x, x_stride, dst, ldd, fz, s, lds, resident);
}

// Q4_0 keeps two steps of weight loads in flight per wave
template <int QT, int M, bool XVEC>
int launch_grp(const uint8_t* W, int64_t N, int64_t K, const float* x, int64_t x_stride,
               float* dst, int64_t ldd, const GemvFuse& fz, hipStream_t s) {
    if constexpr (QT == GQ_TYPE_Q8_0) {
        return launch_grp_pf<QT, M, XVEC, 1>(W, N, K, x, x_stride, dst, ldd, fz, s);
    } else {
        return launch_grp_pf<QT, M, XVEC, 2>(W, N, K, x, x_stride, dst, ldd, fz, s);
    }
}

template <int QT, int M, bool XVEC>
int launch_blk(const uint8_t* W, int64_t N, int64_t K, const float* x, int64_t x_stride,
               float* dst, int64_t ldd, const GemvFuse& fz, hipStream_t s) {
    const int nb = (int)(K / QK);
    const int64_t row_bytes = (int64_t)nb * (QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES);
    const size_t lds = (size_t)M * act_row_bytes(K);
    if (lds > LDS_MAX) return fail(GQ_ERR_UNSUPPORTED, "gemv: activation too large for LDS");
    static size_t allowed = 0;
    int rc = allow_big_lds(&k_gemv_blk<QT, M, XVEC>, allowed, lds);
    if (rc) return rc;
    const dim3 grid((unsigned)cdiv(N, 256 / LPR));
    hipLaunchKernelGGL((k_gemv_blk<QT, M, XVEC>), grid, dim3(256), lds, s, W, N, row_bytes, nb, x,
                       x_stride, dst, ldd, fz);
    return check_hip(hipGetLastError(), "gemv launch");
}

template <int QT, int M>
int launch_m(const uint8_t* W, int64_t N, int64_t K, const float* x, int64_t x_stride, float* dst,
             int64_t ldd, const GemvFuse& fz, hipStream_t s) {
    const bool grp = (K % 256 == 0) && ((reinterpret_cast<uintptr_t>(W) & 15) == 0);
    const bool xvec = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && (x_stride % 4 == 0);
    if (grp)
        return xvec ? launch_grp<QT, M, true>(W, N, K, x, x_stride, dst, ldd, fz, s)
                    : launch_grp<QT, M, false>(W, N, K, x, x_stride, dst, ldd, fz, s);
    return xvec ? launch_blk<QT, M, true>(W, N, K, x, x_stride, dst, ldd, fz, s)
                : launch_blk<QT, M, false>(W, N, K, x, x_stride, dst, ldd, fz, s);
}

template <int QT>
int gemv_t(const uint8_t* W, int64_t N, int64_t K, const float* x, int64_t x_stride, int64_t M,
           float* dst, int64_t ldd, const GemvFuse& fz, hipStream_t s) {
    switch (M) {
        case 1: return launch_m<QT, 1>(W, N, K, x, x_stride, dst, ldd, fz, s);
        case 2: return launch_m<QT, 2>(W, N, K, x, x_stride, dst, ldd, fz, s);
        case 3: return launch_m<QT, 3>(W, N, K, x, x_stride, dst, ldd, fz, s);
        case 4: return launch_m<QT, 4>(W, N, K, x, x_stride, dst, ldd, fz, s);
        default: return fail(GQ_ERR_INVALID, "gemv: M out of range");
    }
}

}  // namespace

int gemv(int type, const uint8_t* W, int64_t N, int64_t K, const float* x, int64_t x_stride,
         int64_t M, float* dst, int64_t ldd, const GemvFuse& fz, hipStream_t s) {
    if (type == GQ_TYPE_Q8_0) return gemv_t<GQ_TYPE_Q8_0>(W, N, K, x, x_stride, M, dst, ldd, fz, s);
    return gemv_t<GQ_TYPE_Q4_0>(W, N, K, x, x_stride, M, dst, ldd, fz, s);
}

}  // namespace gq
