// Prefill GEMM for Q8_0 / Q4_0 weights with exact block products on fp16 MFMA
// (gfx950 v_mfma_f32_32x32x16_f16).
//
// Semantics: ggml_mul_mat with src1 quantized to Q8_0 (llamafile tinyBLAS_Q0 path,
// ggml-cpu/llamafile/sgemm.cpp:3805-4113, entered at ggml-cpu.c:1366-1386):
//   dst[m, n] = sum_b d_w[n, b] * d_x[m, b] * sum_{j<32} q_w[n, b, j] * q_x[m, b, j].
// Every product is formed exactly, and only fp32 accumulation rounds (as on the CPU):
// * the activation quantizer writes d_x * q_x as an exact fp16 pair hi + lo
//   (split_dq8: 18 significant bits over two halves);
// * weight quants are staged in LDS as raw fp16 integers (q, or nibble - 8);
// * per quant block and 32x32 output tile, four MFMAs (hi and lo, two K16 halves)
//   sum sum_j (hi + lo) * q_w, each product exact in fp32 (19 significant bits), into a
//   block accumulator that starts at zero; then acc = fma(d_w, block, acc).
// Against int8 MFMA (v_mfma_i32_32x32x32_i8), which yields the integer block sum in one
// instruction but leaves both scales to VALU (int -> float, d_x * d_w, fma: 3 ops per
// output per block, about 6x the int8 matrix time on CDNA4 without packed fp32), the
// fp16 pair keeps the per-block VALU work to one fma per output and the kernel bound by
// the matrix cores (4 x 32-cycle MFMAs against 16 fmas per lane per block tile).
//
// Tiling: 128 weight rows x BM (128 or 64) tokens per workgroup, K step 64 (two quant
// blocks), 4 waves each owning a BM/2 x 64 sub-tile (MI x 2 MFMA 32x32 tiles). The next
// K steps' global loads are held in a register ring while the current step runs on the
// matrix cores. Quant blocks are loaded with one 16-bit and 8 (Q8_0) or 4 (Q4_0) dword
// loads whose alignment is fixed per block, and expanded with v_perm (0x64xx fp16
// exponent trick) + a packed fp16 subtraction.
#include <algorithm>
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace gq {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int BN = 128, BK = 64, LDK = BK + 8;  // LDS row pitch in halves (144 B)
constexpr int GEMM_PF_128 = 1, GEMM_PF_64 = 2;   // K steps of loads in flight per tile height
#ifndef GEMM_PF_WS
#define GEMM_PF_WS 2  // K steps in the producers' register ring (specialised 128-token kernel)
#endif

__device__ __forceinline__ uint32_t h2_sub_bits(uint32_t pair, half2v bias) {
    half2v h;
    __builtin_memcpy(&h, &pair, 4);
    h = h - bias;  // integers below 2048: exact
    uint32_t r;
    __builtin_memcpy(&r, &h, 4);
    return r;
}

// 4 bytes (values 0..255 as unsigned) -> 4 fp16 of (byte - off), as 2 dwords
__device__ __forceinline__ void expand4(uint32_t u, half2v bias, uint32_t& lo, uint32_t& hi) {
    const uint32_t p01 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t p23 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    lo = h2_sub_bits(p01, bias);
    hi = h2_sub_bits(p23, bias);
}

template <int QT>
struct BlockRegs {
    uint32_t dw[QT == GQ_TYPE_Q8_0 ? 8 : 4];
    uint32_t u;  // the 16-bit piece
    bool even;   // block start is 4-byte aligned
};

constexpr uint32_t OOB = 0x80000000u;  // buffer offset past any resource: reads 0, no fetch

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
    const uint64_t base = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
    const uint32_t n = bytes <= 0 ? 0u : (bytes > 0x7fffffff ? 0x7fffffffu : (uint32_t)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                             (int)__builtin_amdgcn_readfirstlane(n), 0x00020000);
}

// The block at byte offset off of a 4-byte aligned resource, or zeros (scale 0) when not
// `valid`: raw buffer loads, a fixed number per block, so the loads of the register ring
// stay in order for the compiler's memory-counter waits and nothing has to be zeroed
// where the block is used (rows past the resource read 0 as well).
template <int QT>
__device__ __forceinline__ void load_block_rs(__amdgpu_buffer_rsrc_t rs, uint32_t off, bool valid,
                                              BlockRegs<QT>& r) {
    constexpr int NW = QT == GQ_TYPE_Q8_0 ? 8 : 4;
    constexpr uint32_t TAIL = QT == GQ_TYPE_Q8_0 ? 32 : 16;
    r.even = (off & 3) == 0;
    const uint32_t doff = valid ? (r.even ? off : off + 2) : OOB;
    const uint32_t uoff = valid ? (r.even ? off + TAIL : off) : OOB;
#pragma unroll
    for (int i = 0; i < NW; ++i) r.dw[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(doff + 4 * i), 0, 0);
    r.u = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)uoff, 0, 0);
}

// one quant block as its 32 raw quants in fp16 (16 dwords: Q8_0 q, Q4_0 nibble - 8)
// and its scale
template <int QT>
__device__ __forceinline__ void expand_block(const BlockRegs<QT>& r, uint32_t* out, float& d) {
    constexpr int NW = QT == GQ_TYPE_Q8_0 ? 8 : 4;
    uint32_t q[NW];
    uint32_t hdr;
    if (r.even) {
        hdr = r.dw[0] & 0xffffu;
#pragma unroll
        for (int i = 0; i < NW - 1; ++i) q[i] = __builtin_amdgcn_alignbyte(r.dw[i + 1], r.dw[i], 2);
        q[NW - 1] = (r.dw[NW - 1] >> 16) | (r.u << 16);
    } else {
        hdr = r.u;
#pragma unroll
        for (int i = 0; i < NW; ++i) q[i] = r.dw[i];
    }
    d = h2f((uint16_t)hdr);
    if (QT == GQ_TYPE_Q8_0) {
        const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};  // 1024 + 128
#pragma unroll
        for (int i = 0; i < 8; ++i) expand4(q[i] ^ 0x80808080u, bias, out[2 * i], out[2 * i + 1]);
    } else {
        const half2v bias = {(_Float16)1032.0f, (_Float16)1032.0f};  // 1024 + 8
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            expand4(q[i] & 0x0f0f0f0fu, bias, out[2 * i], out[2 * i + 1]);
            expand4((q[i] >> 4) & 0x0f0f0f0fu, bias, out[8 + 2 * i], out[8 + 2 * i + 1]);
        }
    }
}

// BM = 128 or 64 tokens per workgroup (64 doubles the grid of small-N shapes); PF K
// steps of global loads are in flight while a step runs on the matrix cores. A holds
// each token row as 2K halves: the hi parts of d_x * q_x, then the lo parts (lda >= 2K).
//
// Split K (gridDim.z > 1, for grids with fewer tiles than CUs): workgroup z sums K steps
// [z * spk, (z + 1) * spk) and writes its partial tile to part[z][M][N]; k_gemm_reduce
// adds the partials in z order (deterministic).
template <int QT, int BM, int PF>
__global__ __launch_bounds__(256, 2) void k_gemm(const uint8_t* __restrict__ W, int64_t N, int64_t K,
                                                 int64_t row_bytes, const uint16_t* __restrict__ A,
                                                 int64_t lda, int64_t M, float* __restrict__ dst,
                                                 int64_t ldd, int spk, float* __restrict__ part,
                                                 const float* __restrict__ bias, const float* __restrict__ rs) {
    constexpr int BB = QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES;
    constexpr int MI = BM / 64;        // 32-row MFMA tiles per wave along M
    constexpr int AQ = BM / 32;        // 16-byte activation pieces per thread per K step (each of hi, lo)
    __shared__ __align__(16) uint16_t sAh[BM * LDK];
    __shared__ __align__(16) uint16_t sAl[BM * LDK];
    __shared__ __align__(16) uint16_t sB[BN * LDK];
    __shared__ float sD[2][BN];  // weight scales of the K step's two blocks, per weight row
    __shared__ float sRS[BM];    // the tile's activation row scales (read by the epilogue)

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t n0 = (int64_t)blockIdx.x * BN;
    const int64_t m0 = (int64_t)blockIdx.y * BM;
    const int nb = (int)(K / QK);
    const int kt0 = (int)blockIdx.z * spk;
    const int kt1 = min((int)cdiv(K, BK), kt0 + spk);  // this workgroup's K steps [kt0, kt1)

    // loader mapping: B: thread -> (weight row tid / 2, block tid % 2); A: thread ->
    // (token row, AQ consecutive 16-byte pieces of the row's 128-byte K step, hi and lo)
    const int lrow = tid >> 1;
    const int lhalf = tid & 1;
    const int arow = tid / (8 / AQ);
    const int apiece = (tid % (8 / AQ)) * AQ;

    // register ring: PF K steps in flight, raw buffer loads over this workgroup's rows of A
    // and W (rows past M / N, K past the matrix and steps past this split read zeros)
    uint4 rh[PF][AQ], rl[PF][AQ];
    BlockRegs<QT> rb[PF];
    const __amdgpu_buffer_rsrc_t ars = make_rsrc(A + m0 * lda, min<int64_t>(M - m0, BM) * lda * 2);
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(W + n0 * row_bytes, min<int64_t>(N - n0, BN) * row_bytes);
    const uint32_t arow_off = (uint32_t)(arow * lda * 2);
    const uint32_t wrow_off = (uint32_t)(lrow * row_bytes);

    auto load = [&](int kt, int slot) {
        const int64_t k = (int64_t)kt * BK + apiece * 8;
        const bool av = k < K && kt < kt1;
        const uint32_t ao = av ? arow_off + (uint32_t)k * 2 : OOB;
        const uint32_t lo = av ? ao + (uint32_t)K * 2 : OOB;
#pragma unroll
        for (int i = 0; i < AQ; ++i) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(ars, (int)(ao + 16 * i), 0, 0);
            rh[slot][i] = make_uint4(v.x, v.y, v.z, v.w);
        }
#pragma unroll
        for (int i = 0; i < AQ; ++i) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(ars, (int)(lo + 16 * i), 0, 0);
            rl[slot][i] = make_uint4(v.x, v.y, v.z, v.w);
        }
        const int kb = kt * 2 + lhalf;
        load_block_rs<QT>(wrs, wrow_off + (uint32_t)kb * BB, kb < nb && kt < kt1, rb[slot]);
    };

    // the row scales go to LDS with the first step's tiles (the K loop's barriers publish
    // them), so the epilogue needs no memory round trip of its own
    if (tid < BM) sRS[tid] = m0 + tid < M ? rs[m0 + tid] : 1.0f;

    float16v acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // one K step from ring slot `slot`; with PREFETCH the slot is refilled with step kt + PF
    // (always issued, past the matrix from clamped addresses, so every step of the main
    // loop has the same loads in flight and the memory-counter waits stay exact)
    auto step = [&](int kt, int slot, auto prefetch) {
        __syncthreads();  // the previous step's LDS tiles are fully read
        {
            const int ao = arow * LDK + apiece * 8;
            uint4* sah = reinterpret_cast<uint4*>(sAh + ao);
            uint4* sal = reinterpret_cast<uint4*>(sAl + ao);
#pragma unroll
            for (int i = 0; i < AQ; ++i) {
                sah[i] = rh[slot][i];
                sal[i] = rl[slot][i];
            }
            uint32_t e[16];
            float d;
            expand_block<QT>(rb[slot], e, d);  // a zero block: scale 0, quants -8 (Q4_0) or 0
            uint4* sb = reinterpret_cast<uint4*>(sB + lrow * LDK + lhalf * 32);
#pragma unroll
            for (int i = 0; i < 4; ++i) sb[i] = make_uint4(e[4 * i], e[4 * i + 1], e[4 * i + 2], e[4 * i + 3]);
            sD[lhalf][lrow] = d;
        }
        __syncthreads();
        if constexpr (decltype(prefetch)::value) load(kt + PF, slot);
        // MFMA operand layout (32x32x16 f16): lane l holds row l % 32 and the 8 K values
        // 8 (l / 32) .. + 7 of the 16; D[i][j]: column j = l % 32, rows 8 (r / 4) +
        // 4 (l / 32) + r % 4
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {  // the K step's two quant blocks
            const float16v zero = {};
            float16v blk[MI][2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int kk = kb * 32 + h * 16 + 8 * (lane >> 5);
                half8 ah[MI], al[MI], b[2];
#pragma unroll
                for (int i = 0; i < MI; ++i) {
                    const int ro = (wm * (BM / 2) + i * 32 + (lane & 31)) * LDK + kk;
                    ah[i] = *reinterpret_cast<const half8*>(sAh + ro);
                    al[i] = *reinterpret_cast<const half8*>(sAl + ro);
                }
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    b[j] = *reinterpret_cast<const half8*>(sB + (wn * 64 + j * 32 + (lane & 31)) * LDK + kk);
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        blk[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], b[j], h ? blk[i][j] : zero, 0, 0, 0);
                        blk[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], b[j], blk[i][j], 0, 0, 0);
                    }
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float dw = sD[kb][wn * 64 + j * 32 + (lane & 31)];
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(dw, blk[i][j][r], acc[i][j][r]);
            }
        }
    };

#pragma unroll
    for (int p = 0; p < PF; ++p) load(kt0 + p, p);
    int kt = kt0;
    for (; kt + PF <= kt1; kt += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) step(kt + p, p, std::true_type{});
    }
    // tail: the last (kt1 - kt0) % PF steps consume their slots without refilling
#pragma unroll
    for (int p = 0; p < PF - 1; ++p)
        if (kt + p < kt1) step(kt + p, p, std::false_type{});
    if (part) {  // split K: this workgroup's partial tile; the reduce adds the bias
        dst = part + (int64_t)blockIdx.z * M * N;
        ldd = N;
        bias = nullptr;
    }

    // D[i][j]: lane holds column j = lane % 32, rows i = 8*(r/4) + 4*(lane/32) + r%4
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        // the activation rows' power-of-two scales (exact products; 1 for almost every row)
        float rsm[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) rsm[r] = sRS[wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
            if (n >= N) continue;
            const float bn_ = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t m = m0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const float v = acc[i][j][r] * rsm[r];
                if (m < M) dst[m * ldd + n] = bias ? v + bn_ : v;
            }
        }
    }
}

// 128-token tiles with specialised waves: 8 waves per workgroup, one workgroup per CU.
// Waves 4-7 (producers) hold the register ring of global loads, park K step kt + 1 in
// one of two LDS stages and expand its weight blocks, while waves 0-3 (consumers) run
// step kt on the matrix cores from the other stage; one barrier per K step hands the
// stages over. A SIMD then holds one wave of each kind, so the staging work (raw loads,
// weight expansion, LDS writes) overlaps the MFMA phase instead of alternating with it.
// Same tile, operand layout, block products and fma order as k_gemm: same bits.
// The producers stage every step of [kt0, kt1] (kt1 itself reads zeros and is never
// used) and always refill the ring, so their memory-counter waits stay exact.
template <int QT>
constexpr int ws_stage_bytes() {
    return (2 * 128 + BN) * LDK * 2 + 2 * BN * 4;  // sAh, sAl (128 x LDK halves), sB, sD
}

template <int QT, int PF>
__global__ __launch_bounds__(512, 1) void k_gemm_ws(const uint8_t* __restrict__ W, int64_t N, int64_t K,
                                                    int64_t row_bytes, const uint16_t* __restrict__ A,
                                                    int64_t lda, int64_t M, float* __restrict__ dst,
                                                    int64_t ldd, int spk, float* __restrict__ part,
                                                    const float* __restrict__ bias, const float* __restrict__ rs) {
    constexpr int BB = QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES;
    constexpr int BM = 128, MI = 2, AQ = 4;
    constexpr int TILE_H = BM * LDK;  // halves of one of sAh / sAl
    constexpr int STAGE = ws_stage_bytes<QT>();
    extern __shared__ __align__(16) uint8_t gsm[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: role branches are scalar
    const int64_t n0 = (int64_t)blockIdx.x * BN;
    const int64_t m0 = (int64_t)blockIdx.y * BM;
    const int nb = (int)(K / QK);
    const int kt0 = (int)blockIdx.z * spk;
    const int kt1 = min((int)cdiv(K, BK), kt0 + spk);  // this workgroup's K steps [kt0, kt1)

    __shared__ float sRS[BM];  // the tile's activation row scales (read by the consumers' epilogue)
    if (wave >= 4) {
        // producers: thread p -> B: (weight row p / 2, block p % 2); A: (token row p / 2,
        // 16-byte pieces 4 (p % 2) .. + 3 of the row's 128-byte K step, hi and lo)
        const int p = tid - 256;
        if (p < BM) sRS[p] = m0 + p < M ? rs[m0 + p] : 1.0f;  // published by the first barrier
        const int lrow = p >> 1, lhalf = p & 1;
        const int arow = p >> 1, apiece = (p & 1) * AQ;
        uint4 rh[PF][AQ], rl[PF][AQ];
        BlockRegs<QT> rb[PF];
        const __amdgpu_buffer_rsrc_t ars = make_rsrc(A + m0 * lda, min<int64_t>(M - m0, BM) * lda * 2);
        const __amdgpu_buffer_rsrc_t wrs = make_rsrc(W + n0 * row_bytes, min<int64_t>(N - n0, BN) * row_bytes);
        const uint32_t arow_off = (uint32_t)(arow * lda * 2);
        const uint32_t wrow_off = (uint32_t)(lrow * row_bytes);
        auto load = [&](int kt, int slot) {
            const int64_t k = (int64_t)kt * BK + apiece * 8;
            const bool av = k < K && kt < kt1;
            const uint32_t ao = av ? arow_off + (uint32_t)k * 2 : OOB;
            const uint32_t lo = av ? ao + (uint32_t)K * 2 : OOB;
#pragma unroll
            for (int i = 0; i < AQ; ++i) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(ars, (int)(ao + 16 * i), 0, 0);
                rh[slot][i] = make_uint4(v.x, v.y, v.z, v.w);
            }
#pragma unroll
            for (int i = 0; i < AQ; ++i) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(ars, (int)(lo + 16 * i), 0, 0);
                rl[slot][i] = make_uint4(v.x, v.y, v.z, v.w);
            }
            const int kb = kt * 2 + lhalf;
            load_block_rs<QT>(wrs, wrow_off + (uint32_t)kb * BB, kb < nb && kt < kt1, rb[slot]);
        };
        // park ring slot `slot` in LDS stage `buf`
        auto park = [&](int slot, int buf) {
            uint16_t* sAh = reinterpret_cast<uint16_t*>(gsm + buf * STAGE);
            uint16_t* sAl = sAh + TILE_H;
            uint16_t* sB = sAl + TILE_H;
            float* sD = reinterpret_cast<float*>(sB + BN * LDK);
            const int ao = arow * LDK + apiece * 8;
            uint4* sah = reinterpret_cast<uint4*>(sAh + ao);
            uint4* sal = reinterpret_cast<uint4*>(sAl + ao);
#pragma unroll
            for (int i = 0; i < AQ; ++i) {
                sah[i] = rh[slot][i];
                sal[i] = rl[slot][i];
            }
            uint32_t e[16];
            float d;
            expand_block<QT>(rb[slot], e, d);  // a zero block: scale 0, quants -8 (Q4_0) or 0
            uint4* sb = reinterpret_cast<uint4*>(sB + lrow * LDK + lhalf * 32);
#pragma unroll
            for (int i = 0; i < 4; ++i) sb[i] = make_uint4(e[4 * i], e[4 * i + 1], e[4 * i + 2], e[4 * i + 3]);
            sD[lhalf * BN + lrow] = d;
        };
#pragma unroll
        for (int s = 0; s < PF; ++s) load(kt0 + s, s);
        park(0, 0);
        load(kt0 + PF, 0);
        __syncthreads();
        // iteration kt parks step kt + 1 (ring slot (kt + 1 - kt0) % PF) while the
        // consumers run step kt
        auto iter = [&](int kt, int slot) {
            park(slot, (kt + 1 - kt0) & 1);
            load(kt + 1 + PF, slot);
            __syncthreads();
        };
        int kt = kt0;
        for (; kt + PF <= kt1; kt += PF) {
#pragma unroll
            for (int s = 0; s < PF; ++s) iter(kt + s, (s + 1) % PF);
        }
#pragma unroll
        for (int s = 0; s < PF - 1; ++s)
            if (kt + s < kt1) iter(kt + s, (s + 1) % PF);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ring's last (unused) loads
        return;
    }

    // consumers: wave (wm, wn) owns rows wm * 64 .. + 63 of the token tile and weight rows
    // wn * 64 .. + 63
    const int wm = wave >> 1, wn = wave & 1;
    float16v acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    // A K step is 8 tile-blocks (block kb, tile (i, j)), each four dependent MFMAs (hi, lo of
    // two K16 halves) into a block sum. The tiles run in pairs (i, 0), (i, 1) with the two
    // chains interleaved (a dependent MFMA waits for its predecessor's result), and the 32
    // scale fmas of the previous pair run while this pair's 8 MFMAs execute. Each tile keeps
    // its MFMA order and its block order of fmas, so the bits are those of k_gemm.
    // Operand fragments are read one quant block ahead: block 1 of stage kt while block 0
    // runs; after the barrier (stage kt read, stage kt + 1 parked) block 0 of stage kt + 1
    // while block 1 of kt runs.
    const float16v zero = {};
    float16v pend[2] = {zero, zero};  // the pending pair: tiles (1, 0), (1, 1) at a block boundary
    float pdw[2] = {0.0f, 0.0f};      // acc starts at +0, so the first (empty) pending fmas leave it
    struct Frag {
        half8 a[2][MI], l[2][MI], b[2][2];  // [K16 half][i or j]
        float dw[2];
    };
    auto read_block = [&](int stage, int kb, Frag& f) {
        const uint16_t* sAh = reinterpret_cast<const uint16_t*>(gsm + stage * STAGE);
        const uint16_t* sAl = sAh + TILE_H;
        const uint16_t* sB = sAl + TILE_H;
        const float* sD = reinterpret_cast<const float*>(sB + BN * LDK);
        // MFMA operand layout (32x32x16 f16): lane l holds row l % 32 and the 8 K values
        // 8 (l / 32) .. + 7 of the 16; D[i][j]: column j = l % 32, rows 8 (r / 4) +
        // 4 (l / 32) + r % 4
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int kk = kb * 32 + h * 16 + 8 * (lane >> 5);
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int ro = (wm * (BM / 2) + i * 32 + (lane & 31)) * LDK + kk;
                f.a[h][i] = *reinterpret_cast<const half8*>(sAh + ro);
                f.l[h][i] = *reinterpret_cast<const half8*>(sAl + ro);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j)
                f.b[h][j] = *reinterpret_cast<const half8*>(sB + (wn * 64 + j * 32 + (lane & 31)) * LDK + kk);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) f.dw[j] = sD[kb * BN + wn * 64 + j * 32 + (lane & 31)];
    };
    auto run_block = [&](const Frag& f) {
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            float16v blk[2];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    blk[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[h][i], f.b[h][j], h ? blk[j] : zero, 0, 0, 0);
                    blk[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.l[h][i], f.b[h][j], blk[j], 0, 0, 0);
                }
            const int pi = i == 0 ? 1 : 0;  // the pending pair's row of tiles
#pragma unroll
            for (int j = 0; j < 2; ++j) {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[pi][j][r] = __builtin_fmaf(pdw[j], pend[j][r], acc[pi][j][r]);
                pend[j] = blk[j];
                pdw[j] = f.dw[j];
            }
        }
        // one MFMA and four scale fmas at a time
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
    };
    Frag f0, f1;
    __syncthreads();  // stage 0 parked
    read_block(0, 0, f0);
    for (int kt = kt0; kt < kt1; ++kt) {
        const int stage = (kt - kt0) & 1;
        read_block(stage, 1, f1);
        __builtin_amdgcn_sched_barrier(0);  // the reads go out before the block's MFMAs
        run_block(f0);
        __builtin_amdgcn_sched_barrier(0);  // the barrier (and its wait for the reads) after them
        __syncthreads();  // stage kt read; stage kt + 1 parked
        read_block(stage ^ 1, 0, f0);
        __builtin_amdgcn_sched_barrier(0);
        run_block(f1);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[1][j][r] = __builtin_fmaf(pdw[j], pend[j][r], acc[1][j][r]);
    if (part) {  // split K: this workgroup's partial tile; the reduce adds the bias
        dst = part + (int64_t)blockIdx.z * M * N;
        ldd = N;
        bias = nullptr;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        // the activation rows' power-of-two scales (exact products; 1 for almost every row)
        float rsm[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) rsm[r] = sRS[wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
            if (n >= N) continue;
            const float bn_ = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t m = m0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const float v = acc[i][j][r] * rsm[r];
                if (m < M) dst[m * ldd + n] = bias ? v + bn_ : v;
            }
        }
    }
}

// dst[m * ldd + n] = sum_z part[z][m][n], z in order (+ bias[n])
__global__ __launch_bounds__(256) void k_gemm_reduce(const float* __restrict__ part, int ks, int64_t M, int64_t N,
                                                     float* __restrict__ dst, int64_t ldd,
                                                     const float* __restrict__ bias) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= M * N) return;
    const int64_t m = i / N, n = i - m * N;
    float acc = part[i];
    for (int z = 1; z < ks; ++z) acc += part[(int64_t)z * M * N + i];
    dst[m * ldd + n] = bias ? acc + bias[n] : acc;
}

int num_cus() {
    static int ncu = 0;
    if (ncu == 0) {
        int dev = 0, v = 256;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            v = 256;
        ncu = v;
    }
    return ncu;
}

// Tile height: 128 tokens for prompt-sized M on weights of >= 16 row tiles (the grid is
// then filled by splitting K, below); otherwise 128 unless it leaves CUs without a
// workgroup, then 64. (Measured at M = 512, Q4_0: 4096-row o and down projections run
// 14% and 32% faster as 128-token tiles split 4 ways than as unsplit 64-token tiles.)
int gemm_bm(int64_t N, int64_t M) {
    if (M > 64 && cdiv(N, BN) >= 16) return 128;
    return cdiv(N, BN) * cdiv(M, 128) < num_cus() ? 64 : 128;
}

}  // namespace

GemmPlan gemm_plan(int64_t N, int64_t K, int64_t M) {
    GemmPlan p;
    p.bm = gemm_bm(N, M);
    const int64_t ncu = num_cus();
    const int64_t n_tiles = cdiv(N, BN), m_tiles = cdiv(M, p.bm), tiles = n_tiles * m_tiles, nk = cdiv(K, BK);
    // split K while the tiles leave CUs idle, keeping >= 4 K steps per split: up to one
    // workgroup per CU for 128-token tiles (k_gemm_ws holds a CU), two for 64-token tiles
    const int64_t per_cu = p.bm == 128 ? 1 : 2;
    int64_t ks = 1;
    if (tiles < ncu) ks = std::min<int64_t>({cdiv(per_cu * ncu, tiles), nk / 4, 16});
    if (ks < 1) ks = 1;
    p.spk = (int)cdiv(nk, ks);
    p.ks = (int)cdiv(nk, p.spk);  // no empty split
    p.part_bytes = p.ks > 1 ? (size_t)p.ks * M * N * sizeof(float) : 0;
    p.n_head = N, p.ks_tail = 0, p.spk_tail = 0;
    // 128-token tiles over more than one round of CUs: when the last round would be at most
    // half full, its weight rows (whole columns of tiles: a round is ncu / m_tiles columns)
    // run as a second launch with K split so that it fills the CUs (7B qkv at M = 512: 384
    // tiles = 256 + 128, the 128 split 2 ways)
    if (p.bm == 128 && tiles > ncu && ncu % m_tiles == 0) {
        const int64_t per_round = ncu / m_tiles;  // tile columns per round
        const int64_t head = tiles / ncu * per_round;
        const int64_t tail_tiles = (n_tiles - head) * m_tiles;
        if (tail_tiles > 0 && 2 * tail_tiles <= ncu) {
            const int64_t kt = std::min<int64_t>({ncu / tail_tiles, nk / 4, 4});
            if (kt >= 2) {
                p.n_head = head * BN;
                p.spk_tail = (int)cdiv(nk, kt);
                p.ks_tail = (int)cdiv(nk, p.spk_tail);
                p.part_bytes = (size_t)p.ks_tail * M * (N - p.n_head) * sizeof(float);
            }
        }
    }
    return p;
}

namespace {

template <int QT>
int launch(const uint8_t* W, int64_t N, int64_t K, const uint16_t* A, int64_t lda, const float* rs, int64_t M,
           float* dst, int64_t ldd, float* part, hipStream_t s, const float* bias, const GemmPlan& p) {
    const int64_t row_bytes = (K / QK) * (QT == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES);
    float* pp = p.ks > 1 ? part : nullptr;
    if (p.bm == 64) {
        const dim3 grid((unsigned)cdiv(N, BN), (unsigned)cdiv(M, 64), (unsigned)p.ks);
        hipLaunchKernelGGL((k_gemm<QT, 64, GEMM_PF_64>), grid, dim3(256), 0, s, W, N, K, row_bytes, A, lda, M, dst,
                           ldd, p.spk, pp, bias, rs);
    } else {
        constexpr size_t lds = 2 * (size_t)ws_stage_bytes<QT>();  // 112,640 B: two stages
        static_assert(lds <= 160 * 1024, "two stages fit the workgroup's LDS");
        auto* fn = &k_gemm_ws<QT, GEMM_PF_WS>;
        static std::once_flag once;
        static hipError_t attr = hipSuccess;
        std::call_once(once, [&] {
            attr = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
        });
        if (attr != hipSuccess) return check_hip(attr, "gemm: set LDS attribute");
        const dim3 grid((unsigned)cdiv(N, BN), (unsigned)cdiv(M, 128), (unsigned)p.ks);
        hipLaunchKernelGGL(fn, grid, dim3(512), lds, s, W, N, K, row_bytes, A, lda, M, dst, ldd, p.spk, pp, bias, rs);
    }
    int rc = check_hip(hipGetLastError(), "gemm launch");
    if (rc != GQ_OK || p.ks == 1) return rc;
    hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)cdiv(M * N, 256)), dim3(256), 0, s, part, p.ks, M, N, dst, ldd, bias);
    return check_hip(hipGetLastError(), "gemm reduce launch");
}

}  // namespace

int gemm(int type, const uint8_t* W, int64_t N, int64_t K, const uint16_t* A, int64_t lda, const float* rs,
         int64_t M, float* dst, int64_t ldd, float* part, hipStream_t s, const float* bias) {
    if (!rs) return fail(GQ_ERR_INVALID, "gemm: null row scales");
    if ((reinterpret_cast<uintptr_t>(W) & 3) != 0) return fail(GQ_ERR_INVALID, "gemm: weight not 4-byte aligned");
    if ((reinterpret_cast<uintptr_t>(A) & 15) != 0 || lda % 8 != 0 || lda < 2 * K)
        return fail(GQ_ERR_INVALID, "gemm: activation tile misaligned");
    const GemmPlan p = gemm_plan(N, K, M);
    if ((p.ks > 1 || p.ks_tail > 1) && part == nullptr) return fail(GQ_ERR_WORKSPACE, "gemm: split K needs partials");
    auto run = [&](const uint8_t* Wp, int64_t n, float* d, const float* b, const GemmPlan& q) {
        return type == GQ_TYPE_Q8_0 ? launch<GQ_TYPE_Q8_0>(Wp, n, K, A, lda, rs, M, d, ldd, part, s, b, q)
                                    : launch<GQ_TYPE_Q4_0>(Wp, n, K, A, lda, rs, M, d, ldd, part, s, b, q);
    };
    if (p.ks_tail == 0) return run(W, N, dst, bias, p);
    // the whole rounds of tiles, then the tail's weight rows with K split (their own launch,
    // partials and reduce): the same per-tile arithmetic, the tail's sums in split order
    const int64_t row_bytes = (K / QK) * (type == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES);
    GemmPlan head = p;
    head.ks = 1, head.spk = (int)cdiv(K, BK);
    if (int rc = run(W, p.n_head, dst, bias, head)) return rc;
    GemmPlan tail = p;
    tail.ks = p.ks_tail, tail.spk = p.spk_tail;
    return run(W + p.n_head * row_bytes, N - p.n_head, dst + p.n_head, bias ? bias + p.n_head : nullptr, tail);
}

}  // namespace gq
