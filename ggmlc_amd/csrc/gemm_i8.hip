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
#include "epilogue.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace gq {

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));

constexpr int NBS = 8;  // quant blocks per step
constexpr int GEMM_I8_WHOLE_AC = 8;  // 16-byte pieces per thread of the LDS activation copy (32 KiB)
constexpr uint32_t OOB = 0x80000000u;  // buffer offset past any resource: reads 0, no fetch

// Per-wave s_memrealtime stamps of the quantized-SWIGLU launches, compiled only into the
// benchmark's measurement library (GQ_GEMM_STAMPS; libgq has none of this): event e of
// wave w of workgroup x at g_gemm_stamps[(x * 8 + w) * 8 + e]. Events: 0 start, 1 loads
// issued, 2 activation in LDS, 3 first weight step arrived, 4 steps accumulated (1-4 on the
// whole-tile path only), 5 K parts added, 6 the quantized rows' barrier passed, 7 end (0: not
// reached).
#ifdef GQ_GEMM_STAMPS
constexpr int GSTAMP_SLOTS = 2048 * 8 * 8;
__device__ unsigned long long g_gemm_stamps[GSTAMP_SLOTS];
#define GQ_GSTAMP_DECL unsigned long long stamp_[8] = {}
#define GQ_GSTAMP(e)                                          \
    do {                                                      \
        __builtin_amdgcn_sched_barrier(0);                    \
        stamp_[e] = __builtin_amdgcn_s_memrealtime();         \
        __builtin_amdgcn_sched_barrier(0);                    \
    } while (0)
#define GQ_GSTAMP_AFTER(e, x)                                                          \
    do {                                                                               \
        unsigned long long t_;                                                         \
        asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t_) : "v"(x)); \
        stamp_[e] = t_;                                                                \
    } while (0)
#define GQ_GSTAMP_FLUSH()                                                                  \
    do {                                                                                   \
        GQ_GSTAMP(7);                                                                      \
        const size_t i_ = ((size_t)blockIdx.x * 8 + (threadIdx.x >> 6)) * 8;               \
        if ((threadIdx.x & 63) == 0 && i_ + 8 <= (size_t)GSTAMP_SLOTS)                     \
            for (int e_ = 0; e_ < 8; ++e_) g_gemm_stamps[i_ + e_] = stamp_[e_];            \
    } while (0)
#else
#define GQ_GSTAMP_DECL \
    do {               \
    } while (0)
#define GQ_GSTAMP(e) \
    do {             \
    } while (0)
#define GQ_GSTAMP_AFTER(e, x) \
    do {                      \
    } while (0)
#define GQ_GSTAMP_FLUSH() \
    do {                  \
    } while (0)
#endif

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int64_t bytes) {
    const uint64_t base = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
    const uint32_t n = bytes <= 0 ? 0u : (bytes > 0x7fffffff ? 0x7fffffffu : (uint32_t)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                             (int)__builtin_amdgcn_readfirstlane(n), 0x00020000);
}

// Epilogues (template EPI, the I8Epi fusions): plain (+ bias), ROPE + SET_ROWS of a fused
// QKV product, SWIGLU, SWIGLU + the next product's quantized rows. The paired ones read
// logical rows (pair_row): lane l's 4 rows 4 (l / 16) .. + 3 are two whole pairs.
enum { EPI_PLAIN = 0, EPI_ROPE = 1, EPI_GLU = 2, EPI_GLU_Q8 = 3 };

// ORD (KS == 1): the wave sums its K steps in the order of an ORD-part split (part k's
// steps into their own sum, the parts added in part order), so a launch that needs whole
// tiles per workgroup gives the bits of the plan's split launch of the same product.
// NSW > 0 (KS == 1, NSW steps in the row): the workgroup's activation (quants, scales and
// block sums of every block, the workspace bytes as they are) is copied into dynamic LDS
// once, and each wave requests all NSW weight steps of its tile before the first one is
// used: one memory round trip per wave instead of one per step, the registers of the
// per-step activation ring going to the weights. Same operations in the same order as the
// ring, so the same bits.
// KG = 2 (with NSW): workgroups of 8 waves keep the 4 tiles and give each tile's K range to
// 2 waves, whose sums are added in part order through LDS (the bits of a 2-part split):
// two waves per SIMD where a quant block's 4 tiles would otherwise leave one.
// LMH > 0 (ring launches, M <= LMH): the activation rows [0, LMH) of every block are copied
// into dynamic LDS once per workgroup (LAC 16-byte pieces per thread), and the steps take
// their activation operands from there instead of loading them per wave and step (where
// every lane group loads its row's scale and block sum again); the weight ring is unchanged.
// Same operations in the same order, so the same bits.
// SPL: K in two halves (the first ceil(steps / 2) steps, then the rest), each in 4 parts,
// summed as (parts of half 0 in order) + (parts of half 1 in order), every epilogue of a
// gemm_i8_halves product in that order so that fused and unfused chains agree:
//   SPL = 1, KS = 4: one workgroup of 8 waves per tile (KG = 2) adds both halves;
//   SPL = 1, KS = 1 (ORD = 8): one wave walks every step and folds the 8 parts' sums;
//   SPL = 2 (EPI_PLAIN, KS = 4): two workgroups per tile (blockIdx.x & 1 = the half), each
//   writing its half's sum as a slab of dst (half h at dst + h * epi.slab floats); the
//   consumer adds slab 0 + slab 1, which gives the bits of SPL = 1. Narrow products on few
//   workgroups (the configs[4] o and down: 96 row tiles) then stream over twice as many CUs.
template <int QT, int KS, int EPI, int ORD = 1, int NSW = 0, int KG = 1, int LMH = 0, int LAC = 0, int SPL = 0>
__global__ __launch_bounds__(256 * KG, 2 / KG) void k_gemm_i8(const uint8_t* __restrict__ W, int64_t N, int64_t K,
                                                              int64_t row_bytes, const uint8_t* __restrict__ act,
                                                              int64_t M, float* __restrict__ dst, int64_t ldd,
                                                              const float* __restrict__ bias, I8Epi epi) {
    static_assert(NSW == 0 || KS == 1 || LMH > 0, "the whole-tile request of a K part takes the compact copy");
    static_assert(EPI != EPI_GLU_Q8 || KS == 1, "the quantized SWIGLU rows need 4 whole tiles per workgroup");
    static_assert(KG == 1 || (NSW > 0 && ORD == 1) || (SPL == 1 && KS == 4),
                  "8-wave workgroups on the whole-tile path or halves");
    static_assert(SPL == 0 ||
                      (KS == 4 && NSW == 0 && LMH == 0 && ORD == 1 && KG == (SPL == 1 ? 2 : 1) &&
                       (SPL == 1 || EPI == EPI_PLAIN)) ||
                      (KS == 1 && SPL == 1 && ORD == 8 && KG == 1 && LMH == 0),
                  "halves: 4-part ring launches, or the 8-part fold of one-part launches");
    static_assert(LMH == 0 || (KG == 1 && ORD == 1 && (LMH == 8 || LMH == 16) && LAC > 0),
                  "the compact activation copy is for 4-wave launches");
    constexpr int NW = 4 * KG;          // waves per workgroup
    constexpr int PARTS = KS * KG;      // waves per tile (K parts)
    constexpr int BB = QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES;
    constexpr int RB = NBS * BB;           // bytes of a row per step: 272 / 144
    constexpr int CPR = RB / 16;           // 16-byte chunks of a row per step: 17 / 9
    constexpr int CPW = 16 * CPR;          // chunks of a wave's step: 272 / 144
    constexpr int LPL = (CPW + 63) / 64;   // chunk loads per lane per step: 5 / 3
    __shared__ __align__(16) uint8_t s_stage[NW][16 * RB];
    __shared__ float s_red[PARTS > 1 ? NW : 1][64][4];

    GQ_GSTAMP_DECL;
    GQ_GSTAMP(0);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int g = lane >> 4, lr = lane & 15;
    const int tw = wave / PARTS;  // tile of the workgroup
    const int64_t tile = (int64_t)(SPL == 2 ? blockIdx.x >> 1 : blockIdx.x) * (4 / KS) + tw;
    const int kp = wave % PARTS;
    const int64_t n0 = tile * 16;
    const int nb = (int)(K / QK);
    const int nsteps = nb / NBS;
    // the wave's steps [s0, s1): part kp of PARTS, or with halves over the waves (HW) part kh
    // of KS of its half
    constexpr bool HW = SPL != 0 && KS == 4;
    const int half = SPL == 2 ? (int)(blockIdx.x & 1) : (HW ? kp / KS : 0);
    const int kh = HW && SPL == 1 ? kp % KS : kp;
    const int nhs = (nsteps + 1) / 2;  // steps of half 0
    const int hbeg = half * nhs, hend = HW ? min(nsteps, hbeg + nhs) : nsteps;
    const int sp = HW ? (nhs + KS - 1) / KS : (nsteps + PARTS - 1) / PARTS;
    const int s0 = min(hend, hbeg + kh * sp), s1 = min(hend, s0 + sp);

    // the tile's rows of W (rows past N, or a whole tile past N, read 0 without a fetch);
    // paired epilogues: logical row n0 + r is physical row pair_row(n0 + r), the smallest
    // of them pair_row(n0) (N % 16 == 0: tiles are whole)
    constexpr bool PAIRED = EPI != EPI_PLAIN;
    const int64_t rows = N - n0;
    const int64_t pbase = PAIRED && rows > 0 ? pair_row(epi.pair_lo, epi.pair_h, n0) : (rows > 0 ? n0 : 0);
    const int64_t wbytes = rows <= 0 ? 0 : (PAIRED ? (N - pbase) * row_bytes : std::min<int64_t>(rows, 16) * row_bytes);
    const __amdgpu_buffer_rsrc_t wrs = rsrc(W + pbase * row_bytes, wbytes);
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
        const int64_t prow = PAIRED ? pair_row(epi.pair_lo, epi.pair_h, n0 + c / CPR) - pbase : c / CPR;
        coff[i] = cval[i] ? (uint32_t)(prow * row_bytes + (c % CPR) * 16) : 0u;
    }

    auto issue_into = [&](int s, uint4(&wv)[LPL]) {
        const bool live = s < s1;
#pragma unroll
        for (int i = 0; i < LPL; ++i) {
            const uint32_t off = live && cval[i] ? coff[i] + (uint32_t)s * RB : OOB;
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)off, 0, 0);
            wv[i] = make_uint4(v.x, v.y, v.z, v.w);
        }
    };
    uint4 wb[NSW ? 1 : 2][LPL];
    u32x2 ab[NSW ? 1 : 2][NBS];
    float db[NSW ? 1 : 2][NBS];
    int sb[NSW ? 1 : 2][NBS];
    auto issue_w = [&](int s, int slot) { issue_into(s, wb[slot]); };
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
    // the 8 blocks of step s from the parked slice; xop(b, xa, dx, sa) gives block b's
    // activation operand, scale and block sum
    auto blocks = [&](int s, auto xop) {
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
            u32x2 xq;
            float dx;
            int sa;
            xop(b, xq, dx, sa);
            const long xa = (long)(((uint64_t)xq.y << 32) | xq.x);
            const int4v zero = {0, 0, 0, 0};
            const int4v d = __builtin_amdgcn_mfma_i32_16x16x32_i8(wa, xa, zero, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float dw = h2f(*reinterpret_cast<const uint16_t*>(st + (4 * g + r) * RB + b * BB));
                const int isum = QT == GQ_TYPE_Q8_0 ? d[r] : d[r] - 8 * sa;
                acc[r] = __builtin_fmaf((float)isum, dw * dx, acc[r]);
            }
        }
    };
    auto park = [&](const uint4(&wv)[LPL]) {
#pragma unroll
        for (int i = 0; i < LPL; ++i)
            if (cval[i]) *reinterpret_cast<uint4*>(st + (lane + 64 * i) * 16) = wv[i];
        wave_lds_sync();
    };
    // one step from ring slot `slot`: park its weights, refill the slot with step s + 2,
    // then the 8 blocks' MFMAs
    auto body = [&](int s, int slot) {
        park(wb[slot]);
        issue_w(s + 2, slot);
        blocks(s, [&](int b, u32x2& xq, float& dx, int& sa) {
            xq = ab[slot][b];
            dx = db[slot][b];
            sa = QT == GQ_TYPE_Q8_0 ? 0 : sb[slot][b];
        });
        wave_lds_sync();  // the slice is read before the next step parks
        issue_a(s + 2, slot);
    };

    static_assert(ORD == 1 || KS == 1, "the emulated split is for one-part launches");
    float part[ORD][4];
#pragma unroll
    for (int k = 0; k < ORD; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) part[k][r] = 0.0f;
    // first step of part k of the emulated split: k * spo, or with SPL the k % 4-th part of
    // half k / 4 (parts may be empty, their starts then equal: the fold cascades in k order)
    const int spo = SPL ? (nhs + 3) / 4 : (nsteps + ORD - 1) / ORD;
    auto pstart = [&](int k) {
        if constexpr (SPL != 0) return k < 4 ? min(nhs, k * spo) : min(nsteps, nhs + (k - 4) * spo);
        return k * spo;
    };
    auto fold = [&](int st) {  // entering step st: the previous part's sum is complete
        if constexpr (ORD > 1) {
#pragma unroll
            for (int k = 1; k < ORD; ++k)
                if (st == pstart(k)) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) part[k - 1][r] = acc[r], acc[r] = 0.0f;
                }
        }
    };

    // The activation copy into dynamic LDS (whole-tile and staged launches): every thread
    // copies CP pieces of 16 bytes whether or not they hold data (pieces past the data read
    // 0 from the resource and land in the buffer's slack, which the launch sizes to
    // CP * 4096 * KG bytes), since a conditional copy lets the compiler sink a load into
    // the branch, behind the weight loads. Its loads go out before the weight loads and its
    // stores after them, so waiting for the copy leaves the weights in flight.
    // LMH == 0: the workspace bytes as they are (16 rows per block); LMH > 0: the compact
    // copy of rows [0, LMH): quants [nb][LMH][32], scales [nb][LMH] f32, block sums
    // [nb][LMH] i32 (Q4_0), piece q at byte 16 q.
    extern __shared__ __align__(16) uint8_t s_act[];
    constexpr int CP = NSW == 0 && LMH == 0 ? 1 : (LMH ? LAC : GEMM_I8_WHOLE_AC / KG);  // pieces per thread
    constexpr int RH = LMH ? LMH : 16;  // activation rows held per block
    auto copy_issue = [&](u32x4(&av)[CP]) {
        constexpr int QP = RH * 2;  // pieces of a block's quants
        constexpr int SP = RH / 4;  // pieces of a block's scales, and of its block sums
        constexpr int PPB = QP + SP * (QT == GQ_TYPE_Q4_0 ? 2 : 1);
        const int nq = nb * QP, ns = nb * SP;
        const __amdgpu_buffer_rsrc_t ars = rsrc(act, (int64_t)nb * (QT == GQ_TYPE_Q4_0 ? 640 : 576));
#pragma unroll
        for (int i = 0; i < CP; ++i) {
            const int q = (int)threadIdx.x + 256 * KG * i;
            uint32_t off = (uint32_t)q * 16;
            if constexpr (LMH > 0) {
                if (q < nq) off = (uint32_t)((q / QP) * 512 + (q % QP) * 16);
                else if (q < nq + ns) off = (uint32_t)(nb * 512 + ((q - nq) / SP) * 64 + ((q - nq) % SP) * 16);
                else off = (uint32_t)(nb * 576 + ((q - nq - ns) / SP) * 64 + ((q - nq - ns) % SP) * 16);
                if (q >= nb * PPB) off = OOB;
            }
            av[i] = __builtin_amdgcn_raw_buffer_load_b128(ars, (int)off, 0, 0);
        }
    };
    auto copy_store = [&](const u32x4(&av)[CP]) {
#pragma unroll
        for (int i = 0; i < CP; ++i)
            *reinterpret_cast<u32x4*>(s_act + ((int)threadIdx.x + 256 * KG * i) * 16) = av[i];
    };
    const int lra = RH == 16 ? lr : (lr & (RH - 1));  // rows past RH (past M) read row lr - RH
    // step s's activation operands from the copy
    auto lds_blocks = [&](int s) {
        blocks(s, [&](int b, u32x2& xq, float& dx, int& sa) {
            const int e = (s * NBS + b) * RH + lra;  // (block, activation row)
            xq = *reinterpret_cast<const u32x2*>(s_act + e * 32 + 8 * g);
            dx = *reinterpret_cast<const float*>(s_act + nb * RH * 32 + e * 4);
            sa = QT == GQ_TYPE_Q8_0 ? 0 : *reinterpret_cast<const int*>(s_act + nb * RH * 36 + e * 4);
        });
    };

    if constexpr (NSW > 0) {
        // the activation into LDS, every weight step of the wave, then the steps in order
        // as their loads return
        u32x4 av[CP];
        copy_issue(av);
        __builtin_amdgcn_sched_barrier(0);
        uint4 wr[NSW][LPL];
#pragma unroll
        for (int j = 0; j < NSW; ++j) issue_into(s0 + j, wr[j]);
        __builtin_amdgcn_sched_barrier(0);
        GQ_GSTAMP(1);
        copy_store(av);
        __syncthreads();
        GQ_GSTAMP(2);
        GQ_GSTAMP_AFTER(3, wr[0][0].x);
#pragma unroll
        for (int j = 0; j < NSW; ++j) {
            const int s = s0 + j;
            if (s >= s1) break;  // uniform
            fold(s);
            park(wr[j]);
            lds_blocks(s);
            wave_lds_sync();  // the slice is read before the next step parks
        }
        GQ_GSTAMP_AFTER(4, acc[0]);
    } else if constexpr (LMH > 0) {
        // the activation into LDS, then the two-step weight ring
        u32x4 av[CP];
        copy_issue(av);
        __builtin_amdgcn_sched_barrier(0);
        issue_w(s0, 0);
        issue_w(s0 + 1, 1);
        __builtin_amdgcn_sched_barrier(0);
        copy_store(av);
        __syncthreads();
        auto body_l = [&](int s, int slot) {
            park(wb[slot]);
            issue_w(s + 2, slot);
            lds_blocks(s);
            wave_lds_sync();  // the slice is read before the next step parks
        };
        int s = s0;
        for (; s + 1 < s1; s += 2) {
            body_l(s, 0);
            body_l(s + 1, 1);
        }
        if (s < s1) body_l(s, 0);
    } else {
        issue_w(s0, 0);
        issue_a(s0, 0);
        issue_w(s0 + 1, 1);
        issue_a(s0 + 1, 1);
        int s = s0;
        for (; s + 1 < s1; s += 2) {
            fold(s);
            body(s, 0);
            fold(s + 1);
            body(s + 1, 1);
        }
        if (s < s1) {
            fold(s);
            body(s, 0);
        }
    }
    if constexpr (ORD > 1) {  // the last part's sum, then the parts in order (empty ones 0)
        int kl = 0;  // the part of the last step
#pragma unroll
        for (int k = 1; k < ORD; ++k)
            if (pstart(k) <= s1 - 1) kl = k;
#pragma unroll
        for (int k = 0; k < ORD; ++k)
            if (k == kl) {
#pragma unroll
                for (int r = 0; r < 4; ++r) part[k][r] = acc[r];
            }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if constexpr (SPL != 0) {  // (half 0's parts in order) + (half 1's parts in order)
                float a0 = part[0][r], a1 = part[4][r];
#pragma unroll
                for (int k = 1; k < 4; ++k) a0 += part[k][r], a1 += part[4 + k][r];
                acc[r] = a0 + a1;
            } else {
                acc[r] = part[0][r];
#pragma unroll
                for (int k = 1; k < ORD; ++k) acc[r] += part[k][r];
            }
        }
    }

    // the tile's K parts added in part order in its first wave; with the quantized SWIGLU
    // rows the other waves stay for the epilogue's barriers
    const bool first = kp == 0;
    if constexpr (PARTS > 1) {
#pragma unroll
        for (int r = 0; r < 4; ++r) s_red[wave][lane][r] = acc[r];
        __syncthreads();
        if (EPI != EPI_GLU_Q8 && !first) return;
        if constexpr (HW && SPL == 1) {  // (half 0's parts in order) + (half 1's parts in order)
            float a1[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) a1[r] = s_red[wave + KS][lane][r];
#pragma unroll
            for (int k = 1; k < KS; ++k)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    acc[r] += s_red[wave + k][lane][r];
                    a1[r] += s_red[wave + KS + k][lane][r];
                }
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] += a1[r];
        } else {
#pragma unroll
            for (int k = 1; k < PARTS; ++k)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] += s_red[wave + k][lane][r];
        }
    }
    GQ_GSTAMP_AFTER(5, acc[0]);
    const int64_t m = lr;  // activation row
    if constexpr (EPI == EPI_PLAIN) {
        if (m >= M) return;
        float* const dh = SPL == 2 ? dst + half * epi.slab : dst;  // this half's slab
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t n = n0 + 4 * g + r;
            if (n < N) dh[m * ldd + n] = bias ? acc[r] + bias[n] : acc[r];
        }
    } else {
        // the lane's two pairs: logical rows (row, row + 1), row = n0 + 4 g + 2 p; the bias is
        // added to the product first, at the physical rows (v + bias: ADD(MUL_MAT, bias))
        float v[2], vp[2];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int64_t row = n0 + 4 * g + 2 * p;
            v[p] = acc[2 * p];
            vp[p] = acc[2 * p + 1];
            if (bias && n0 < N) {
                v[p] = v[p] + bias[pair_row(epi.pair_lo, epi.pair_h, row)];
                vp[p] = vp[p] + bias[pair_row(epi.pair_lo, epi.pair_h, row + 1)];
            }
        }
        if constexpr (EPI == EPI_ROPE) {
            if (m >= M || n0 >= N) return;
            const GemvRope& r = epi.rp;
            const int64_t kv = r.idx[m];
            auto cs = [&](int c) {
                if (r.cache) return *reinterpret_cast<const float2*>(reinterpret_cast<const uint8_t*>(r.cache) +
                                                                     m * r.cache_nb1 + (int64_t)c * 8);
                float co, si;
                rope_cs((float)r.pos[m], c, r.theta_scale, r.freq_scale, r.attn_factor, co, si);
                return make_float2(co, si);
            };
#pragma unroll
            for (int p = 0; p < 2; ++p) rope_store(r, (int)m, kv, n0 + 4 * g + 2 * p, v[p], vp[p], cs);
        } else {
            float u[2];
#pragma unroll
            for (int p = 0; p < 2; ++p) u[p] = swiglu_f(v[p], vp[p]);
            if (first && dst && m < M && n0 < N) {
#pragma unroll
                for (int p = 0; p < 2; ++p) dst[m * ldd + (n0 >> 1) + 2 * g + p] = u[p];
            }
            if constexpr (EPI == EPI_GLU_Q8) {
                // one quant block per workgroup: SWIGLU outputs 32 b .. + 31 (b = blockIdx.x)
                // of every activation row, 8 per wave, 2 per lane (rows of the same m sit in
                // lanes lr, lr + 16, lr + 32, lr + 48 of each wave); quantize_row_q8_0's rule
                // on the block max and the exact integer block sum, as quant8_block
                __shared__ float s_amax[4][16];
                __shared__ int s_isum[4][16];
                float a = fmaxf(fabsf(u[0]), fabsf(u[1]));
                a = fmaxf(a, __shfl_xor(a, 16, 64));
                a = fmaxf(a, __shfl_xor(a, 32, 64));
                if (first && g == 0) s_amax[tw][lr] = a;
                __syncthreads();
                float amax = s_amax[0][lr];
#pragma unroll
                for (int w = 1; w < 4; ++w) amax = fmaxf(amax, s_amax[w][lr]);
                const float d = amax / 127.0f;
                const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
                int q[2];
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const int iv = (int)__builtin_rintf(u[p] * id);
                    q[p] = iv > 127 ? 127 : (iv < -128 ? -128 : iv);
                }
                int is = q[0] + q[1];
                is += __shfl_xor(is, 16, 64);
                is += __shfl_xor(is, 32, 64);
                if (first && g == 0) s_isum[tw][lr] = is;
                __syncthreads();
                GQ_GSTAMP(6);
                if (!first || m >= M || n0 >= N) {
                    GQ_GSTAMP_FLUSH();
                    return;
                }
                const int64_t nbq = N / 64;  // blocks of the quantized rows (K = N / 2)
                const int64_t e = (int64_t)blockIdx.x * 16 + m;  // (block, activation row)
                *reinterpret_cast<uint16_t*>(epi.q8 + e * 32 + 8 * tw + 2 * g) =
                    (uint16_t)((q[0] & 0xff) | ((q[1] & 0xff) << 8));
                if (tw == 0 && g == 0) {
                    int isum = s_isum[0][lr];
#pragma unroll
                    for (int w = 1; w < 4; ++w) isum += s_isum[w][lr];
                    *reinterpret_cast<float*>(epi.q8 + nbq * 512 + e * 4) = h2f(f2h(d));
                    *reinterpret_cast<int*>(epi.q8 + nbq * 576 + e * 4) = isum;
                }
                GQ_GSTAMP_FLUSH();
            }
        }
    }
}

// One-part launches of rows of WHOLE_STEPS steps (K = 1536: the configs[4] gate|up and
// output head) request each wave's whole tile at once, the activation staged in LDS
// (measured on the configs[4] shapes; GQ_OPT_GEMM_I8_RING keeps the per-step ring)
constexpr int WHOLE_STEPS = 6;
static_assert(GEMM_I8_WHOLE_AC * 4096 >= WHOLE_STEPS * NBS * 640, "the LDS copy covers the activation bytes");

template <int QT, int EPI, int ORD, int KG = 1, int SPL = 0>
int launch_whole(const dim3& g, const uint8_t* W, int64_t N, int64_t K, int64_t row_bytes, const uint8_t* act,
                 int64_t M, float* dst, int64_t ldd, hipStream_t s, const float* bias, const I8Epi& e) {
    const size_t lds = (size_t)GEMM_I8_WHOLE_AC * 4096;  // every thread's pieces, data or not
    hipLaunchKernelGGL((k_gemm_i8<QT, 1, EPI, ORD, WHOLE_STEPS / KG, KG, 0, 0, SPL>), g, dim3(256 * KG), lds, s, W,
                       N, K, row_bytes, act, M, dst, ldd, bias, e);
    return check_hip(hipGetLastError(), "gemm_i8 launch");
}

// Ring launches of up to 8 rows with 2 or 4 tiles per workgroup and the activation staged
// in LDS (LMH = 8): LAC = 10 pieces of 16 bytes per thread hold the compact copy of K <= 4096
// (20 pieces per block for Q4_0, 18 for Q8_0: 40 KB). Measured at M = 8 (configs[1], Q4_0):
// gate_up 22016 x 4096 (2 K parts) 26.0 -> 21.7 us. One-tile workgroups (4 K parts) re-read
// nothing within the workgroup and were slower staged (Qwen2.5-1.5B o at M = 8: 5.4 -> 5.8 us;
// down, K = 8960, with a 112 KB copy: 11.7 -> 12.4 us).
template <int QT, int KS, int LAC>
int launch_lact(const dim3& g, const uint8_t* W, int64_t N, int64_t K, int64_t row_bytes, const uint8_t* act,
                int64_t M, float* dst, int64_t ldd, hipStream_t s, const float* bias, const I8Epi& e) {
    hipLaunchKernelGGL((k_gemm_i8<QT, KS, EPI_PLAIN, 1, 0, 1, 8, LAC>), g, dim3(256), (size_t)LAC * 4096, s, W, N, K,
                       row_bytes, act, M, dst, ldd, bias, e);
    return check_hip(hipGetLastError(), "gemm_i8 launch");
}

template <int QT, int EPI>
int launch_epi(const uint8_t* W, int64_t N, int64_t K, const uint8_t* act, int64_t M, float* dst, int64_t ldd,
               hipStream_t s, const float* bias, const I8Epi& e) {
    const int64_t row_bytes = (K / QK) * (QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES);
    const GemmI8Plan p = gemm_i8_plan(N, K);
    const bool whole = K / (QK * NBS) == WHOLE_STEPS && !option_gemm_i8_ring();
    if constexpr (EPI == EPI_GLU_Q8) {  // one quant block (64 logical rows) per workgroup,
        // summed in the order of the plan's split (the bits of the unfused product)
        const dim3 g((unsigned)(N / 64));
        const bool hv = gemm_i8_halves(N, K);  // the 8 parts of K's two halves
        if (whole) {
            if (hv) return launch_whole<QT, EPI, 8, 1, 1>(g, W, N, K, row_bytes, act, M, dst, ldd, s, bias, e);
            if (p.ks == 4) return launch_whole<QT, EPI, 4>(g, W, N, K, row_bytes, act, M, dst, ldd, s, bias, e);
            // the 2-part split as 8-wave workgroups (two waves per tile)
            if (p.ks == 2) return launch_whole<QT, EPI, 1, 2>(g, W, N, K, row_bytes, act, M, dst, ldd, s, bias, e);
            return launch_whole<QT, EPI, 1>(g, W, N, K, row_bytes, act, M, dst, ldd, s, bias, e);
        }
        if (hv)
            hipLaunchKernelGGL((k_gemm_i8<QT, 1, EPI, 8, 0, 1, 0, 0, 1>), g, dim3(256), 0, s, W, N, K, row_bytes, act,
                               M, dst, ldd, bias, e);
        else if (p.ks == 4)
            hipLaunchKernelGGL((k_gemm_i8<QT, 1, EPI, 4>), g, dim3(256), 0, s, W, N, K, row_bytes, act, M, dst, ldd,
                               bias, e);
        else if (p.ks == 2)
            hipLaunchKernelGGL((k_gemm_i8<QT, 1, EPI, 2>), g, dim3(256), 0, s, W, N, K, row_bytes, act, M, dst, ldd,
                               bias, e);
        else
            hipLaunchKernelGGL((k_gemm_i8<QT, 1, EPI, 1>), g, dim3(256), 0, s, W, N, K, row_bytes, act, M, dst, ldd,
                               bias, e);
        return check_hip(hipGetLastError(), "gemm_i8 launch");
    }
    const dim3 grid((unsigned)p.wgs);
    if (p.ks == 1 && whole) return launch_whole<QT, EPI, 1>(grid, W, N, K, row_bytes, act, M, dst, ldd, s, bias, e);
    if constexpr (EPI == EPI_PLAIN) {
        if (M <= 8 && p.ks <= 2 && (K / QK) * (QT == GQ_TYPE_Q4_0 ? 20 : 18) <= 10 * 256 && !option_gemm_i8_ring()) {
            if (p.ks == 2) return launch_lact<QT, 2, 10>(grid, W, N, K, row_bytes, act, M, dst, ldd, s, bias, e);
            return launch_lact<QT, 1, 10>(grid, W, N, K, row_bytes, act, M, dst, ldd, s, bias, e);
        }
    }
    if (gemm_i8_halves(N, K)) {
        if (EPI == EPI_PLAIN && e.slab)  // two workgroups per tile, one per half, each writing its own slab
            hipLaunchKernelGGL((k_gemm_i8<QT, 4, EPI_PLAIN, 1, 0, 1, 0, 0, 2>), dim3((unsigned)(2 * p.wgs)), dim3(256),
                               0, s, W, N, K, row_bytes, act, M, dst, ldd, bias, e);
        else  // both halves in one 8-wave workgroup per tile: their sum in the same order, then the epilogue
            hipLaunchKernelGGL((k_gemm_i8<QT, 4, EPI == EPI_GLU_Q8 ? EPI_GLU : EPI, 1, 0, 2, 0, 0, 1>), grid, dim3(512),
                               0, s, W, N, K, row_bytes, act, M, dst, ldd, bias, e);
        return check_hip(hipGetLastError(), "gemm_i8 launch");
    }
    if (p.ks == 4)
        hipLaunchKernelGGL((k_gemm_i8<QT, 4, EPI == EPI_GLU_Q8 ? EPI_GLU : EPI>), grid, dim3(256), 0, s, W, N, K,
                           row_bytes, act, M, dst, ldd, bias, e);
    else if (p.ks == 2)
        hipLaunchKernelGGL((k_gemm_i8<QT, 2, EPI == EPI_GLU_Q8 ? EPI_GLU : EPI>), grid, dim3(256), 0, s, W, N, K,
                           row_bytes, act, M, dst, ldd, bias, e);
    else
        hipLaunchKernelGGL((k_gemm_i8<QT, 1, EPI>), grid, dim3(256), 0, s, W, N, K, row_bytes, act, M, dst, ldd,
                           bias, e);
    return check_hip(hipGetLastError(), "gemm_i8 launch");
}

template <int QT>
int launch(const uint8_t* W, int64_t N, int64_t K, const uint8_t* act, int64_t M, float* dst, int64_t ldd,
           hipStream_t s, const float* bias, const I8Epi* e) {
    const I8Epi none{};
    if (!e || (!e->rope && !e->glu)) return launch_epi<QT, EPI_PLAIN>(W, N, K, act, M, dst, ldd, s, bias, e ? *e : none);
    if (e->rope) return launch_epi<QT, EPI_ROPE>(W, N, K, act, M, dst, ldd, s, bias, *e);
    if (e->q8) return launch_epi<QT, EPI_GLU_Q8>(W, N, K, act, M, dst, ldd, s, bias, *e);
    return launch_epi<QT, EPI_GLU>(W, N, K, act, M, dst, ldd, s, bias, *e);
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

// measured at 16 rows on the Qwen2.5-1.5B shapes (96 row tiles), two workgroups per tile
// against one: down (K = 8960) 11.76 -> 8.48 us, o (K = 1536) 5.28 -> 4.76 us; a CU streams
// at most ~20 GB/s, so a launch of fewer workgroups than CUs is bound by its workgroup count
bool gemm_i8_halves(int64_t N, int64_t K) { return gemm_i8_plan(N, K).ks == 4 && cdiv(N, 16) <= 128; }

int gemm_i8(int type, const uint8_t* W, int64_t N, int64_t K, const uint8_t* act, int64_t M, float* dst,
            int64_t ldd, hipStream_t s, const float* bias, const I8Epi* epi) {
    if (K % GEMM_I8_K_ALIGN != 0 || M < 1 || M > GEMM_I8_MAX_M)
        return fail(GQ_ERR_INVALID, "gemm_i8: needs K % 256 == 0 and 1 <= M <= 16");
    if ((reinterpret_cast<uintptr_t>(W) & 15) != 0 || (reinterpret_cast<uintptr_t>(act) & 15) != 0)
        return fail(GQ_ERR_INVALID, "gemm_i8: weight and activation must be 16-byte aligned");
    if (epi && (epi->rope || epi->glu)) {
        const int64_t row_bytes = (K / QK) * (type == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES);
        if (N % (epi->glu && epi->q8 ? 64 : 16) != 0)
            return fail(GQ_ERR_UNSUPPORTED, "gemm_i8: paired epilogues need N % 16 == 0 (64 with quantized rows)");
        if (N * row_bytes > 0x7fffffffLL) return fail(GQ_ERR_UNSUPPORTED, "gemm_i8: paired epilogues need < 2 GiB weights");
        if (epi->rope && epi->pair_lo != 0 && (epi->pair_lo + 1) % 16 != 0)
            return fail(GQ_ERR_UNSUPPORTED, "gemm_i8: NEOX rope epilogue needs head_dim % 16 == 0");
        if (epi->q8 && (reinterpret_cast<uintptr_t>(epi->q8) & 15) != 0)
            return fail(GQ_ERR_INVALID, "gemm_i8: quantized rows must be 16-byte aligned");
    }
    if (epi && epi->slab && (epi->rope || epi->glu || bias || !gemm_i8_halves(N, K)))
        return fail(GQ_ERR_INVALID, "gemm_i8: two output halves only for products gemm_i8_halves splits, no bias");
    if (type == GQ_TYPE_Q8_0) return launch<GQ_TYPE_Q8_0>(W, N, K, act, M, dst, ldd, s, bias, epi);
    return launch<GQ_TYPE_Q4_0>(W, N, K, act, M, dst, ldd, s, bias, epi);
}

}  // namespace gq
