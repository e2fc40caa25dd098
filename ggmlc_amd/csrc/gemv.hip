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
#include <type_traits>
#include <unordered_map>

#include "common.h"
#include "epilogue.h"
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
// block (a0, a1 = its 32 int8; sa = their sum); Q4_0 nibbles are dotted unsigned
// and biased by 8 through the block sum, so the block sum stays an exact integer
template <int QT>
__device__ __forceinline__ int block_dot(const uint32_t* q, const uint4& a0, const uint4& a1, int sa) {
    if constexpr (QT == GQ_TYPE_Q8_0) {
        (void)sa;
        int s = dot4(q[0], a0.x, 0);
        s = dot4(q[1], a0.y, s);
        s = dot4(q[2], a0.z, s);
        s = dot4(q[3], a0.w, s);
        s = dot4(q[4], a1.x, s);
        s = dot4(q[5], a1.y, s);
        s = dot4(q[6], a1.z, s);
        return dot4(q[7], a1.w, s);
    } else {
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

// sum over the 16 lanes of a row (DPP within rows of 16 lanes: every lane ends
// with the row total; pairs, quads, half-row mirror, row mirror)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    return v;
}

// Physical weight row of logical row r (pair_row: rows of a wave are 4 consecutive logical
// rows, so both rows of a SWIGLU / rope pair land in one wave)
__device__ __forceinline__ int64_t phys_row(const GemvFuse& fz, int64_t r) {
    return pair_row(fz.pair_lo, fz.pair_h, r);
}

// (cos, sin) of every rotated pair of the M positions (tab[m * n_dims/2 + j]) and
// the M cache rows (after the pairs), computed once per workgroup into LDS while
// the first weight loads are in flight
// With a rope cache (the (cos, sin) table of the M positions, gq_rope_cache) each
// thread holds at most RC of its entries; larger tables are computed here.
constexpr int RC = 2;
template <int M>
struct RopeIn {
    int32_t pos[M];
    int64_t row[M];
    float2 cs[RC];
};
__device__ __forceinline__ bool rope_cached(const GemvFuse& fz, int M) {
    return fz.rope && fz.rp.cache && M * (fz.rp.n_dims >> 1) <= RC * 256;
}
// the cached (cos, sin) entries of this thread: raw buffer loads issued whether or not
// the launch uses them (an empty resource returns 0 without a fetch), so the vector
// memory counter stays exact for the weight loads issued after them
template <int M>
__device__ __forceinline__ void rope_cache_loads(const GemvFuse& fz, RopeIn<M>& in) {
    const bool use = rope_cached(fz, M);
    const int np = fz.rp.n_dims >> 1;
    const uint64_t base = reinterpret_cast<uint64_t>(fz.rp.cache);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
    const uint32_t n = use ? (uint32_t)(M * fz.rp.cache_nb1) : 0u;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0, (int)__builtin_amdgcn_readfirstlane(n),
        0x00020000);
#pragma unroll
    for (int k = 0; k < RC; ++k) {
        const int idx = (int)threadIdx.x + k * (int)blockDim.x;  // the entries rope_table stores
        const int m = use ? idx / np : 0, j = idx - m * np;
        const uint32_t off = use && idx < M * np ? (uint32_t)(m * fz.rp.cache_nb1 + j * 8) : 0x80000000u;
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)off, 0, 0);
        in.cs[k] = make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
    }
}
// the cache rows and, when the (cos, sin) table is not cached, the positions
// (wave-uniform loads), read first thing; nothing waits for them before the weight
// loads are issued
template <int M>
__device__ __forceinline__ void rope_inputs(const GemvFuse& fz, RopeIn<M>& in) {
#pragma unroll
    for (int m = 0; m < M; ++m) in.row[m] = fz.rp.idx[m];
    if (!rope_cached(fz, M)) {
#pragma unroll
        for (int m = 0; m < M; ++m) in.pos[m] = fz.rp.pos[m];
    }
}
// (cos, sin) of every rotated pair of the M positions (tab[m * n_dims/2 + j]) and the
// M cache rows (after the pairs) into LDS
template <int M>
__device__ __forceinline__ void rope_table(const GemvFuse& fz, const RopeIn<M>& in, float2* tab) {
    const GemvRope& r = fz.rp;
    const int np = r.n_dims >> 1;
    if (rope_cached(fz, M)) {
#pragma unroll
        for (int k = 0; k < RC; ++k) {
            const int idx = (int)threadIdx.x + k * (int)blockDim.x;
            if (idx < M * np) tab[idx] = in.cs[k];
        }
    } else {
        for (int idx = threadIdx.x; idx < M * np; idx += blockDim.x) {
            const int m = idx / np, j = idx - m * np;
            int32_t p = in.pos[0];
#pragma unroll
            for (int mm = 1; mm < M; ++mm) p = m == mm ? in.pos[mm] : p;
            float c, s;
            rope_cs((float)p, j, r.theta_scale, r.freq_scale, r.attn_factor, c, s);
            tab[idx] = make_float2(c, s);
        }
    }
    if (threadIdx.x == 0) {
#pragma unroll
        for (int m = 0; m < M; ++m) reinterpret_cast<int64_t*>(tab + M * np)[m] = in.row[m];
    }
}

// Rope epilogue from the LDS table: (cos, sin) of row m's pairs and its cache row
template <int M>
__device__ __forceinline__ void rope_emit(const GemvRope& r, const float2* tab, int m, int64_t row, float v0,
                                          float v1) {
    const int64_t kv = reinterpret_cast<const int64_t*>(tab + M * (r.n_dims >> 1))[m];
    rope_store(r, m, kv, row, v0, v1, [&](int c) { return tab[m * (r.n_dims >> 1) + c]; });
}

// Write logical row `row` of activation m: plain, residual-added (res + v: the
// operand order of ADD(x, MUL_MAT)), or, for the paired epilogues (SWIGLU, rope),
// from the even row with its partner's value vp. A bias is added to the product first
// (v + bias: the operand order of ADD(MUL_MAT, bias), executor.cpp:2436-2445).
template <int M>
__device__ __forceinline__ void emit(const GemvFuse& fz, const float2* rtab, float* dst, int64_t ldd, int m,
                                     int64_t row, float v, float vp) {
    if (fz.bias) {
        v = v + fz.bias[phys_row(fz, row)];
        if (fz.glu | fz.rope) vp = vp + fz.bias[phys_row(fz, row ^ 1)];
    }
    if (fz.glu) {
        if ((row & 1) == 0) dst[(int64_t)m * ldd + (row >> 1)] = swiglu_f(v, vp);
        return;
    }
    if (fz.rope) {
        if ((row & 1) == 0) rope_emit<M>(fz.rp, rtab, m, row, v, vp);
        return;
    }
    if (fz.res) v = fz.res[(int64_t)m * fz.ldr + row] + v;
    dst[(int64_t)m * ldd + row] = v;
}

template <int QT, int M, bool XVEC, int PF, int KS, int XPT, int PRE>
__global__ __launch_bounds__(256, 2) void k_gemv_grp(const uint8_t* __restrict__ W, int64_t N,
                                                     int64_t row_bytes, int G, ActSrc act, float* dst,
                                                     int64_t ldd, GemvFuse fz) {
    constexpr int GB = QTraits<QT>::GB;
    constexpr int CPG = QTraits<QT>::CPG;
    constexpr int SEG = LPR * CPG;       // chunks of one row per step
    constexpr int XPMAX = 6;             // activation passes held in registers (K <= 12288 at M = 1)
    constexpr int XAMAX = 2;             // of which can carry a fused ADD operand
    // XPT > 0: the launch has exactly XPT activation passes (M = 1), so the prologue's
    // passes are straight-line code the compiler can interleave
    static_assert(XPT == 0 || (M == 1 && XPT <= XPMAX), "exact pass count only for one row");
    constexpr int XPN = XPT ? XPT : XPMAX;
    constexpr int RG = WAVES / KS;       // row groups (of RPW rows) per workgroup tile
    constexpr int ROWS = RG * RPW;       // rows per workgroup tile
    constexpr uint32_t OOB = 0x80000000u;  // buffer offset past any matrix: load returns 0, no fetch
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float red[WAVES][M][RPW];
    __shared__ double red_d[4];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int act_bytes = G * ACT_GS;
    uint8_t* s_act = smem;
    uint8_t* s_stage = smem + M * act_bytes + wave * 64 * GB;
    float2* rtab = reinterpret_cast<float2*>(smem + M * act_bytes + WAVES * 64 * GB);  // rope epilogue only

    const int rsub = lane / LPR;
    const int gsub = lane % LPR;
    const int nb = G * 8;
    const int XP = XPT ? XPT : (nb * 4 + 255) / 256;

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

    // persistent workgroups over workgroup tiles of ROWS rows; each wave walks its
    // (tile, step) sequence with a PF-deep register pipeline. (Measured: contiguous
    // per-wave row ranges sized N / waves, which balance bytes exactly, ran slower:
    // partial row sets cost more steps.)
    const int64_t n_wgt = (N + ROWS - 1) / ROWS;
    const int my_wgt = blockIdx.x < n_wgt ? (int)((n_wgt - blockIdx.x + gridDim.x - 1) / gridDim.x) : 0;

    // activation loads first, then the weight prefetch: the activation can then be
    // waited for while the weight loads stay in flight (vector loads complete in order)
    RopeIn<M> rin{};
    rope_cache_loads<M>(fz, rin);
    if (fz.rope) rope_inputs<M>(fz, rin);
    float xr[XPMAX][8], ar[XAMAX][8];
    const bool xpre = M * XP <= XPMAX && (!act.d || M * XP <= XAMAX);
    if (xpre) {
#pragma unroll
        for (int p = 0; p < XPN; ++p) {
            if (XPT || p < M * XP) {
                const int m = p / XP, t = (p - m * XP) * 256 + (int)threadIdx.x;
                load8<XVEC>(act.x + (int64_t)m * act.xs + (int64_t)t * 8, (t >> 2) < nb, xr[p]);
                if (p < XAMAX && act.d)
                    load8<XVEC>(act.d + (int64_t)m * act.ds + (int64_t)t * 8, (t >> 2) < nb, ar[p]);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // Weight loads are raw buffer loads: per step one wave-uniform base (the step's
    // 4-row slice at its first group) plus a per-lane constant offset, so a load costs
    // no address arithmetic. Offsets past the resource's size return 0 without a
    // memory access: rows past N, chunks past the K range of a tail step and steps
    // past the end of the wave's sequence never touch memory.
    // Chunk c of a lane is byte 16 * within of slice row r (r, within from lane + 64 c);
    // with paired rows (phys_row) slice rows 2i, 2i+1 are physical rows i and i + pair_h
    // past the slice's first physical row (a slice never straddles a pair block: blocks
    // are the whole matrix or a multiple of 4 rows).
    const int64_t mat_bytes = N * row_bytes;
    uint32_t voff[CPG];
#pragma unroll
    for (int c = 0; c < CPG; ++c) {
        const int ci = lane + 64 * c, r = ci / SEG, within = ci - r * SEG;
        const int64_t roff = fz.pair_lo ? (int64_t)(r >> 1) + (r & 1) * fz.pair_h : (int64_t)r;
        voff[c] = (uint32_t)(roff * row_bytes + within * 16);
    }
    const int ngr_tail = g_end - g_begin - (S - 1) * LPR;  // groups of the last step of a tile
    uint4 pre[PF][CPG];
    // load cursor: tile k, step j (wave-uniform)
    int lk = 0, lj = 0;
    // chunks [LO, HI) of the step at the load cursor; the cursor moves on when ADV (a step may
    // be issued in two parts, both for the same cursor position)
    auto issue_rng = [&](uint4(&buf)[CPG], auto lo_c, auto hi_c, bool adv) {
        constexpr int LO = decltype(lo_c)::value, HI = decltype(hi_c)::value;
        const int64_t row0 = ((int64_t)blockIdx.x + (int64_t)lk * gridDim.x) * ROWS + rg * RPW;
        const int64_t prow = phys_row(fz, row0);
        const int gfirst = g_begin + lj * LPR;
        const int64_t off0 = prow * row_bytes + (int64_t)gfirst * GB;
        const int64_t left = lk < my_wgt ? mat_bytes - off0 : 0;
        const uint32_t nrec = left <= 0 ? 0u : (left > 0x7fffffff ? 0x7fffffffu : (uint32_t)left);
        // the resource lives in SGPRs: make its wave-uniformity explicit
        const uint64_t base = reinterpret_cast<uint64_t>(W) + (uint64_t)off0;
        const uint32_t blo = __builtin_amdgcn_readfirstlane((uint32_t)base);
        const uint32_t bhi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
        __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            reinterpret_cast<void*>(((uint64_t)bhi << 32) | blo), (short)0,
            (int)__builtin_amdgcn_readfirstlane(nrec), 0x00020000);
        const bool tail = lj == S - 1 && ngr_tail < LPR;
#pragma unroll
        for (int c = 0; c < CPG; ++c) {
            if (c < LO || c >= HI) continue;  // resolved at compile time
            uint32_t vo = voff[c];
            if (tail) {  // chunks of groups past the K range
                const int ci = lane + 64 * c, within = ci - (ci / SEG) * SEG;
                vo = within < ngr_tail * CPG ? vo : OOB;
            }
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)vo, 0, 2 /* nt */);
            buf[c] = make_uint4(v.x, v.y, v.z, v.w);
        }
        if (adv && ++lj == S) lj = 0, ++lk;
    };
    using C0 = std::integral_constant<int, 0>;
    using CP = std::integral_constant<int, CPG>;
    auto issue = [&](uint4(&buf)[CPG]) { issue_rng(buf, C0{}, CP{}, true); };
    // the first step's loads (its first PRE chunks when PRE < CPG) go out before the
    // activation prologue, the rest after it: a CU serves its waves' memory requests in
    // order, so an activation load issued behind many weight loads holds the prologue
    // (measured: 5-13% faster launches; the partial first step for grids of a tile or more
    // per resident workgroup: 7B qkv, gate_up and lm_head 4-12% faster)
    issue_rng(pre[0], C0{}, std::integral_constant<int, PRE>{}, false);
    __builtin_amdgcn_sched_barrier(0);
    if (fz.rope) rope_table<M>(fz, rin, rtab);  // while the loads are in flight

    float scale[M];
#pragma unroll
    for (int m = 0; m < M; ++m) scale[m] = 1.0f;
    if (xpre) {
        if (act.d) {  // ADD fused in front: x + d, stored once for the nodes that read the sum
#pragma unroll
            for (int p = 0; p < XAMAX; ++p) {
                if (p < XPN && (XPT || p < M * XP)) {
                    const int m = p / XP, t = (p - m * XP) * 256 + (int)threadIdx.x;
#pragma unroll
                    for (int i = 0; i < 8; ++i) xr[p][i] = xr[p][i] + ar[p][i];
                    act_store_sum<XVEC>(act, blockIdx.x == 0, m, (int64_t)t * 8, (t >> 2) < nb, xr[p]);
                }
            }
        }
        if (fz.rms) {  // RMS_NORM fused: the rows' squares are already in registers
#pragma unroll
            for (int m = 0; m < M; ++m) {
                double sq = 0.0;
#pragma unroll
                for (int p = 0; p < XPN; ++p)
                    if ((XPT || p < M * XP) && p / XP == m) sq = sumsq8(xr[p], sq);
                scale[m] = rms_scale(block_sum_d(sq, red_d), (int64_t)G * 256, fz.eps);
            }
        }
#pragma unroll
        for (int p = 0; p < XPN; ++p) {
            if (XPT || p < M * XP) {  // uniform across the workgroup
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
                    if (part == 0)
                        *reinterpret_cast<float2*>(gp + ACT_DS_OFF + 8 * bi) =
                            make_float2(h2f(dh), __int_as_float(qsum));
                }
            }
        }
    } else {
        if (fz.rms) rms_scales<XVEC, M>(act, M, G * 256, fz.eps, scale, red_d);
        quantize_rows_to_act<XVEC, M>(act, blockIdx.x == 0, M, G * 256, s_act, act_bytes, scale);
    }
    __syncthreads();  // quantized activation (and rope table) visible to all waves
    issue_rng(pre[0], std::integral_constant<int, PRE>{}, CP{}, true);  // nothing when PRE == CPG
#pragma unroll
    for (int s = 1; s < PF; ++s) issue(pre[s]);

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;

    // consume cursor: tile k, step j (wave-uniform)
    int ck = 0, cj = 0;
    // One step: park buffer `buf` in the wave's LDS slice, refill it with the step PF
    // ahead, decode. The PF buffers are used round-robin by an unrolled loop so no
    // register copy of a pending load forces an early wait.
    auto body = [&](uint4(&buf)[CPG]) {
        const int64_t row = ((int64_t)blockIdx.x + (int64_t)ck * gridDim.x) * ROWS + rg * RPW + rsub;
#pragma unroll
        for (int c = 0; c < CPG; ++c) *reinterpret_cast<uint4*>(s_stage + (lane + 64 * c) * 16) = buf[c];
        wave_lds_sync();
        issue(buf);
        const int g = g_begin + cj * LPR + gsub;
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
            for (int m = 0; m < M; ++m) {
                const uint8_t* ag = s_act + m * act_bytes + g * ACT_GS;
                const float4 ds01 = *reinterpret_cast<const float4*>(ag + ACT_DS_OFF + 32 * h);
                const float4 ds23 = *reinterpret_cast<const float4*>(ag + ACT_DS_OFF + 32 * h + 16);
                const float dsv[8] = {ds01.x, ds01.y, ds01.z, ds01.w, ds23.x, ds23.y, ds23.z, ds23.w};
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) {
                    const int b = 4 * h + bb;
                    uint32_t hdr;
                    uint32_t q[QTraits<QT>::NQW];
                    decode_at<QT>(w, QTraits<QT>::BB * b - 16 * c0, hdr, q);
                    const float dw = h2f((uint16_t)hdr);
                    const uint4 a0 = *reinterpret_cast<const uint4*>(ag + ACT_QS_OFF + 32 * b);
                    const uint4 a1 = *reinterpret_cast<const uint4*>(ag + ACT_QS_OFF + 32 * b + 16);
                    const int sdot = block_dot<QT>(q, a0, a1, __float_as_int(dsv[2 * bb + 1]));
                    acc[m] += (float)sdot * (dw * dsv[2 * bb]);
                }
            }
        }
        wave_lds_sync();  // this step's staging slice is fully read before it is refilled
        if (cj == S - 1) {  // tile finished: reduce the 16 lanes of each row, then the K parts
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float v = row16_sum(acc[m]);
                acc[m] = 0.0f;
                if constexpr (KS == 1) {
                    float vp = 0.0f;
                    if (fz.glu | fz.rope) vp = __shfl_xor(v, LPR, 64);  // the next row's value (pairs)
                    if (gsub == 0 && row < N) emit<M>(fz, rtab, dst, ldd, m, row, v, vp);
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
                        emit<M>(fz, rtab, dst, ldd, m, row, v, vp);
                    }
                }
                __syncthreads();
            }
        }
        if (++cj == S) cj = 0, ++ck;
    };
    const int F = my_wgt * S;
    if constexpr (PF == 1) {
        for (int f = 0; f < F; ++f) body(pre[0]);
    } else {
        static_assert(PF == 2, "prefetch depth 1 or 2");
        int f = 0;
        for (; f + 1 < F; f += 2) {
            body(pre[0]);
            body(pre[1]);
        }
        if (f < F) body(pre[0]);
    }
}

// ---- fallback: one lane per block, 16-bit loads (any K % 32 == 0) ---------------

template <int QT, int M, bool XVEC>
__global__ __launch_bounds__(256) void k_gemv_blk(const uint8_t* __restrict__ W, int64_t N,
                                                  int64_t row_bytes, int nb, ActSrc act, float* dst,
                                                  int64_t ldd, GemvFuse fz) {
    constexpr int BB = QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES;
    constexpr int NQW = QT == GQ_TYPE_Q8_0 ? 8 : 4;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red_d[4];
    const int act_stride = (int)act_row_bytes((int64_t)nb * QK);
    const uint8_t* s_act = smem;
    float scale[M];
#pragma unroll
    for (int m = 0; m < M; ++m) scale[m] = 1.0f;
    if (fz.rms) rms_scales<XVEC, M>(act, M, nb * QK, fz.eps, scale, red_d);
    quantize_rows_to_act<XVEC, M>(act, blockIdx.x == 0, M, nb * QK, smem, act_stride, scale);
    float2* rtab = reinterpret_cast<float2*>(smem + M * act_stride);  // rope epilogue only
    if (fz.rope) {
        RopeIn<M> rin{};
        rope_cache_loads<M>(fz, rin);
        rope_inputs<M>(fz, rin);
        rope_table<M>(fz, rin, rtab);
    }
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
                const uint8_t* ag = s_act + m * act_stride + (int64_t)g * ACT_GS;
                const uint4 a0 = *reinterpret_cast<const uint4*>(ag + ACT_QS_OFF + 32 * bi);
                const uint4 a1 = *reinterpret_cast<const uint4*>(ag + ACT_QS_OFF + 32 * bi + 16);
                const float2 ds = *reinterpret_cast<const float2*>(ag + ACT_DS_OFF + 8 * bi);
                const float da = ds.x;
                const int s = block_dot<QT>(q, a0, a1, __float_as_int(ds.y));
                acc[m] += (float)s * (dw * da);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float v = row16_sum(acc[m]);
        const float vp = __shfl_xor(v, LPR, 64);
        if (sub == 0 && row < N) emit<M>(fz, rtab, dst, ldd, m, row, v, vp);
    }
}

constexpr size_t LDS_MAX = 160 * 1024;

// LDS of the rope epilogue's (cos, sin) table
size_t rope_lds(const GemvFuse& fz, int64_t M) {
    return fz.rope ? (size_t)M * (fz.rp.n_dims / 2) * sizeof(float2) + (size_t)M * sizeof(int64_t) : 0;
}

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

template <int QT, int M, bool XVEC, int PF, int KS, int XPT, int PRE = QTraits<QT>::CPG>
int launch_grp_ks(const uint8_t* W, int64_t N, int64_t K, const ActSrc& act,
                  float* dst, int64_t ldd, const GemvFuse& fz, hipStream_t s, size_t lds, int resident) {
    const int G = (int)(K / 256);
    const int64_t row_bytes = (K / QK) * QTraits<QT>::BB;
    auto* fn = &k_gemv_grp<QT, M, XVEC, PF, KS, XPT, PRE>;
    static size_t allowed = 0;
    int rc = allow_big_lds(fn, allowed, lds);
    if (rc) return rc;
    const int64_t tiles = cdiv(N, (WAVES / KS) * RPW);
    // persistent grid with the same number of tiles per workgroup (768 qkv tiles over 512
    // resident workgroups: 384 x 2 instead of 1.5 on average; measured 0.3% on tg128)
    const int64_t per = cdiv(tiles, resident);
    const dim3 grid((unsigned)(tiles < resident ? tiles : cdiv(tiles, per)));
    hipLaunchKernelGGL(fn, grid, dim3(256), lds, s, W, N, row_bytes, G, act, dst, ldd, fz);
    return check_hip(hipGetLastError(), "gemv launch");
}

template <int QT, int M, bool XVEC, int PF, int XPT>
int launch_grp_pf(const uint8_t* W, int64_t N, int64_t K, const ActSrc& act,
                  float* dst, int64_t ldd, const GemvFuse& fz, hipStream_t s) {
    const int G = (int)(K / 256);
    const size_t lds = (size_t)M * G * ACT_GS + (size_t)WAVES * 64 * QTraits<QT>::GB + rope_lds(fz, M);
    if (lds > LDS_MAX) return fail(GQ_ERR_UNSUPPORTED, "gemv: activation too large for LDS");
    // residency is the same for every KS (same registers and LDS)
    int resident = 0;
    int rc = resident_wgs(&k_gemv_grp<QT, M, XVEC, PF, 1, XPT, QTraits<QT>::CPG>, lds, resident);
    if (rc) return rc;
    // split K over the waves of a workgroup (whole steps per wave) only when
    // the row tiles leave most CUs without a workgroup (measured: splitting a
    // 4096-row down projection is slower, a 1536-row one faster)
    const int64_t t1 = cdiv(N, WAVES * RPW);
    const int J = (G + LPR - 1) / LPR;
    // one row, a tile or more per resident workgroup: only part of the first step goes out
    // before the activation prologue (4 of 9 chunks for Q4_0, 8 of 17 for Q8_0)
    if constexpr (M == 1) {
        if (t1 >= resident)
            return launch_grp_ks<QT, M, XVEC, PF, 1, XPT, QT == GQ_TYPE_Q8_0 ? 8 : 4>(W, N, K, act, dst, ldd, fz, s,
                                                                                       lds, resident);
    }
    if (4 * t1 >= resident || J < 2)
        return launch_grp_ks<QT, M, XVEC, PF, 1, XPT>(W, N, K, act, dst, ldd, fz, s, lds, resident);
    if (J < 3) return launch_grp_ks<QT, M, XVEC, PF, 2, XPT>(W, N, K, act, dst, ldd, fz, s, lds, resident);
    return launch_grp_ks<QT, M, XVEC, PF, 4, XPT>(W, N, K, act, dst, ldd, fz, s, lds, resident);
}

// Q4_0 keeps two steps of weight loads in flight per wave
template <int QT, int M, bool XVEC, int XPT>
int launch_grp_x(const uint8_t* W, int64_t N, int64_t K, const ActSrc& act,
                 float* dst, int64_t ldd, const GemvFuse& fz, hipStream_t s) {
    if constexpr (QT == GQ_TYPE_Q8_0) {
        return launch_grp_pf<QT, M, XVEC, 1, XPT>(W, N, K, act, dst, ldd, fz, s);
    } else {
        return launch_grp_pf<QT, M, XVEC, 2, XPT>(W, N, K, act, dst, ldd, fz, s);
    }
}

// one-row launches with 16-byte aligned activations get the instance with their exact
// number of prologue passes (K = 1536, 2560-4096, 8960-10240, 10496-12288: the
// configs' shapes); the rest the generic one
template <int QT, int M, bool XVEC>
int launch_grp(const uint8_t* W, int64_t N, int64_t K, const ActSrc& act,
               float* dst, int64_t ldd, const GemvFuse& fz, hipStream_t s) {
    if constexpr (M == 1 && XVEC) {
        switch (cdiv(K / QK * 4, 256)) {
            case 1: return launch_grp_x<QT, M, XVEC, 1>(W, N, K, act, dst, ldd, fz, s);
            case 2: return launch_grp_x<QT, M, XVEC, 2>(W, N, K, act, dst, ldd, fz, s);
            case 5: return launch_grp_x<QT, M, XVEC, 5>(W, N, K, act, dst, ldd, fz, s);
            case 6: return launch_grp_x<QT, M, XVEC, 6>(W, N, K, act, dst, ldd, fz, s);
            default: break;
        }
    }
    return launch_grp_x<QT, M, XVEC, 0>(W, N, K, act, dst, ldd, fz, s);
}

template <int QT, int M, bool XVEC>
int launch_blk(const uint8_t* W, int64_t N, int64_t K, const ActSrc& act,
               float* dst, int64_t ldd, const GemvFuse& fz, hipStream_t s) {
    const int nb = (int)(K / QK);
    const int64_t row_bytes = (int64_t)nb * (QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES);
    const size_t lds = (size_t)M * act_row_bytes(K) + rope_lds(fz, M);
    if (lds > LDS_MAX) return fail(GQ_ERR_UNSUPPORTED, "gemv: activation too large for LDS");
    static size_t allowed = 0;
    int rc = allow_big_lds(&k_gemv_blk<QT, M, XVEC>, allowed, lds);
    if (rc) return rc;
    const dim3 grid((unsigned)cdiv(N, 256 / LPR));
    hipLaunchKernelGGL((k_gemv_blk<QT, M, XVEC>), grid, dim3(256), lds, s, W, N, row_bytes, nb, act, dst, ldd,
                       fz);
    return check_hip(hipGetLastError(), "gemv launch");
}

inline bool vec_ok(const float* p, int64_t stride) {
    return p == nullptr || (((reinterpret_cast<uintptr_t>(p) & 15) == 0) && (stride % 4 == 0));
}

template <int QT, int M>
int launch_m(const uint8_t* W, int64_t N, int64_t K, const ActSrc& act, float* dst, int64_t ldd,
             const GemvFuse& fz, hipStream_t s) {
    const bool grp = (K % 256 == 0) && ((reinterpret_cast<uintptr_t>(W) & 15) == 0);
    const bool xvec = vec_ok(act.x, act.xs) && vec_ok(act.d, act.ds) && vec_ok(act.out, act.os);
    if (grp)
        return xvec ? launch_grp<QT, M, true>(W, N, K, act, dst, ldd, fz, s)
                    : launch_grp<QT, M, false>(W, N, K, act, dst, ldd, fz, s);
    return xvec ? launch_blk<QT, M, true>(W, N, K, act, dst, ldd, fz, s)
                : launch_blk<QT, M, false>(W, N, K, act, dst, ldd, fz, s);
}

template <int QT>
int gemv_t(const uint8_t* W, int64_t N, int64_t K, const ActSrc& act, int64_t M, float* dst, int64_t ldd,
           const GemvFuse& fz, hipStream_t s) {
    switch (M) {
        case 1: return launch_m<QT, 1>(W, N, K, act, dst, ldd, fz, s);
        case 2: return launch_m<QT, 2>(W, N, K, act, dst, ldd, fz, s);
        case 3: return launch_m<QT, 3>(W, N, K, act, dst, ldd, fz, s);
        case 4: return launch_m<QT, 4>(W, N, K, act, dst, ldd, fz, s);
        default: return fail(GQ_ERR_INVALID, "gemv: M out of range");
    }
}

}  // namespace

int gemv(int type, const uint8_t* W, int64_t N, int64_t K, const ActSrc& act, int64_t M, float* dst, int64_t ldd,
         const GemvFuse& fz, hipStream_t s) {
    if (type == GQ_TYPE_Q8_0) return gemv_t<GQ_TYPE_Q8_0>(W, N, K, act, M, dst, ldd, fz, s);
    return gemv_t<GQ_TYPE_Q4_0>(W, N, K, act, M, dst, ldd, fz, s);
}

}  // namespace gq
