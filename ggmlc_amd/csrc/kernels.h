// Internal launchers (host side) implemented by the .hip files of libgq.
#pragma once

#include "common.h"

namespace gq {

// api.hip: process-wide switches set through gq_set_option
bool option_attn_separate_merge();
bool option_gemm_i8_ring();

// quantize.hip
int quantize_q8_0_blocks(const float* x, int64_t nrows, int64_t K, int64_t x_stride, void* y,
                         hipStream_t s);
// The GEMM path's fused activation prologue (quantize.hip): per row of x (row stride xs),
// x + d (stored to sum when given) or SWIGLU of the row's halves (glu: x rows are 2K
// wide), then RMS_NORM (rms), then d * q of quantize_row_q8_0 into y as the exact fp16
// pair hi + lo of d * q / rs[m] (split_dq8): hi at y[m * y_stride + k], lo at
// y[m * y_stride + K + k] (y_stride >= 2K), rs[m] the row's power-of-two scale that keeps
// hi finite (row_pow2; 1 unless the row's amax passes ~65500), which the GEMM multiplies
// back. quantize_q8_0_f16 writes the same without the neighbours (two launches: the row
// scales, then the blocks).
constexpr int64_t PREP_MAX_K = 16384;
struct ActPrep {
    const float* x;
    int64_t xs;
    const float* d;
    int64_t ds;
    float* sum;
    int64_t ss;
    int64_t K;
    int rms, glu;
    float eps;
    const float* d2 = nullptr;  // with d: v = x + (d + d2), d2's rows at the stride ds
};
int act_prep(const ActPrep& a, int64_t M, uint16_t* y, int64_t y_stride, float* rs, hipStream_t s);
// The same prologue for gemm_i8 (M <= 16): the quants of quantize_row_q8_0 as int8 in
// the i8 layout, per block b: y[b * 512 + m * 32 + j] the quants of row m, then
// y[nb * 512 + (b * 16 + m) * 4] the scale (f32) and y[nb * 576 + (b * 16 + m) * 4] the
// block sum (i32); gemm_i8_act_bytes(K) bytes
int act_prep_i8(const ActPrep& a, int64_t M, uint8_t* y, hipStream_t s);
int quantize_q8_0_f16(const float* x, int64_t nrows, int64_t K, int64_t x_stride, uint16_t* y,
                      int64_t y_stride_elems, float* rs, hipStream_t s);
int quantize_weights(int type, const float* x, void* y, int64_t n, hipStream_t s);

// gemv.hip — dst[m * ldd + n] for m < M (M <= GEMV_MAX_M); x fp32 rows (stride x_stride),
// quantized inside the kernel
constexpr int GEMV_MAX_M = 4;
// Fusions of the decoder graph's neighbours of MUL_MAT into the GEMV (each gives the
// bits of the unfused ops): ADD in front of the activation (ActSrc.d), RMS_NORM of
// the activation rows, SWIGLU over the two halves of the weight rows (output N/2
// wide), ADD of a residual to the output (may alias dst).
// ROPE of the q and k rows plus SET_ROWS of k and v, applied to the rows of a fused
// QKV product ((Hq + 2 Hkv) heads of hd rows): the work of k_rope_kv as an epilogue
struct GemvRope {
    const int32_t* pos;   // [M] positions
    const float* cache;   // [M][n_dims/2][2] (cos, sin) of the positions, or null: computed here
    int64_t cache_nb1;    // bytes per position
    int64_t hd, Hq, Hkv;
    int hd_log2;          // hd is a power of two
    int n_dims, neox;
    float theta_scale, freq_scale, attn_factor;
    float* qo;
    int64_t qonb1, qonb2;  // bytes per head, per token
    uint16_t* kc;
    int64_t kcnb1, kcnb2;  // bytes per cache row, per head
    uint16_t* vc;
    int64_t vcnb1, vcnb2;
    int64_t rows;
    const int64_t* idx;  // [M] cache rows
    int32_t* n_bad;
};

// Fusions of the decode GEMV. Paired epilogues see logical rows 2c, 2c+1 in one
// wave: with pair_lo != 0 (a block of pair_lo + 1 rows, a power of two >= 4, or
// all ones for one block) logical row r reads physical row
//   (r & ~pair_lo) + ((r & pair_lo) >> 1) + (r & 1) * pair_h
// (SWIGLU: pair_lo = ~0, pair_h = N/2, gate row c with up row c + N/2; NEOX rope:
// pair_lo = hd - 1, pair_h = hd/2, dims c and c + hd/2 of a head; normal rope
// pairs adjacent dims: pair_lo = 0, the identity).
struct GemvFuse {
    int rms = 0;
    float eps = 0.0f;
    int glu = 0;
    int rope = 0;
    int64_t pair_lo = 0, pair_h = 0;
    const float* res = nullptr;
    int64_t ldr = 0;
    const float* bias = nullptr;  // [N] added to the product first (MUL_MAT's bias ADD)
    GemvRope rp{};
};
int gemv(int type, const uint8_t* W, int64_t N, int64_t K, const ActSrc& act, int64_t M, float* dst, int64_t ldd,
         const GemvFuse& fz, hipStream_t s);

// gemm.hip — dst[m * ldd + n] = rs[m] * sum_k A[m * lda + k] * dequant(W)[n, k] (+ bias[n]),
// A the fp16 hi + lo rows of the activation prologue and rs its row scales; grids with fewer
// tiles than CUs split K over ks workgroups whose partials (part, part_bytes) are summed in
// order by a second kernel
struct GemmPlan {
    int bm, ks, spk;
    size_t part_bytes;
    // a last round of 128-token tiles that would leave at least half the CUs idle: the
    // weight rows from n_head on run as a second launch with K split ks_tail ways
    // (0: no tail launch)
    int64_t n_head;
    int ks_tail, spk_tail;
};
GemmPlan gemm_plan(int64_t N, int64_t K, int64_t M);
int gemm(int type, const uint8_t* W, int64_t N, int64_t K, const uint16_t* A, int64_t lda, const float* rs,
         int64_t M, float* dst, int64_t ldd, float* part, hipStream_t s, const float* bias = nullptr);

// gemm_i8.hip — dst[m * ldd + n] for 1 <= M <= GEMM_I8_MAX_M activation rows on int8
// MFMA, for K % 256 == 0 and 16-byte aligned weights, from act_prep_i8's layout; 16-row
// tiles, the 4 waves of a workgroup splitting K into ks parts for narrow weights
constexpr int GEMM_I8_MAX_M = 16;
constexpr int64_t GEMM_I8_K_ALIGN = 256;
inline size_t gemm_i8_act_bytes(int64_t K) { return (size_t)(K / 32) * 640; }
struct GemmI8Plan {
    int ks;
    int64_t wgs;
};
GemmI8Plan gemm_i8_plan(int64_t N, int64_t K);
// plain products of at most 128 row tiles in 4 K parts take K in two halves (the sum of
// half 0, then of half 1, then half 0 + half 1, then the bias): one 8-wave workgroup per
// tile, or without a bias and with I8Epi::slab two workgroups per tile writing one half
// each for the consumer to add
bool gemm_i8_halves(int64_t N, int64_t K);
// Output-side fusions of gemm_i8 (the GEMV's, on the same logical row pairs: pair_row):
//   rope: ROPE + SET_ROWS of a fused QKV product (rp; dst unused), N % 16 == 0;
//   glu: SWIGLU of the pairs (gate row c, up row c + N/2) into dst[m * ldd + c] (dst may be
//     null), N % 64 == 0; with q8, also those rows quantized (quantize_row_q8_0) into q8 in
//     act_prep_i8's layout for K = N/2 — what the next product's prologue would write.
struct I8Epi {
    int rope = 0, glu = 0;
    int64_t pair_lo = 0, pair_h = 0;
    GemvRope rp{};
    uint8_t* q8 = nullptr;
    int64_t slab = 0;  // gemm_i8_halves products: half h's sum at dst + h * slab floats (0: their sum at dst)
};
int gemm_i8(int type, const uint8_t* W, int64_t N, int64_t K, const uint8_t* act, int64_t M, float* dst,
            int64_t ldd, hipStream_t s, const float* bias = nullptr, const I8Epi* epi = nullptr);

// set_rows.hip
struct SetRowsArgs {
    uint16_t* dst;
    int64_t ne0, ne1, ne2, ne3;   // dst shape
    int64_t dnb1, dnb2, dnb3;     // dst byte strides
    const float* src;
    int64_t s;                    // src rows (ne1 of src)
    int64_t snb1, snb2, snb3;     // src byte strides
    const void* idx;
    int idx64;
    int64_t ine1, ine2;           // idx broadcast extents
    int64_t inb0, inb1, inb2;     // idx byte strides
    int32_t* n_bad;
};
int set_rows_f32_f16(const SetRowsArgs& a, hipStream_t s);

// attention.hip
struct AttnArgs {
    const float* q;
    int64_t D, S, Hq, Hkv;
    int64_t qnb1, qnb2;           // bytes
    const uint16_t* k;
    const uint16_t* v;
    int64_t n_kv;
    int64_t knb1, knb2, vnb1, vnb2;  // bytes
    const uint16_t* mask;          // may be null
    int64_t mnb1;                  // bytes
    float scale, max_bias, softcap;
    float* dst;                    // [S][Hq][D]
};
size_t attn_workspace_bytes(int64_t D, int64_t S, int64_t Hq, int64_t Hkv, int64_t n_kv);
int attention(const AttnArgs& a, void* ws, size_t ws_bytes, hipStream_t s);
int attn_reset_counters(hipStream_t s);
// the same launches with the split partials in a static per-device array of
// ATTN_SCRATCH_BYTES (no workspace); attn_scratch_init looks its address up once per
// device (the current one) and returns it
constexpr size_t ATTN_SCRATCH_BYTES = (size_t)16 << 20;
int attn_scratch_init(void** out);
int attention_noalloc(const AttnArgs& a, hipStream_t s);
// batched decode over a paged KV pool: sequence b has len[b] rows, logical row r at pool
// row table[b * tstride + (r >> log2p)] << log2p | (r & (2^log2p - 1))
struct PagedKv {
    const int32_t* len;
    const int32_t* table;
    int64_t tstride;
    int log2p;
    int B;
};
// a.q: [B][Hq][D] rows (qnb1 = sequence stride, qnb2 = head stride), a.n_kv = pool rows,
// a.dst [B][Hq][D]; max_len bounds every len[b] (sizes the grid)
size_t attn_paged_workspace_bytes(int64_t D, int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len, int64_t page);
// q8: with the matrix-core kernel and a split merge (B <= 16), the output rows also
// quantized in act_prep_i8's layout (K = Hq * D) by the merge; ignored otherwise
int attention_paged(const AttnArgs& a, const PagedKv& pg, int64_t max_len, void* ws, size_t ws_bytes, hipStream_t s,
                    uint8_t* q8 = nullptr);
// whether attention_paged with q8 writes it: the matrix-core kernel with a split merge
bool attention_paged_q8_ok(int64_t D, int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len, int64_t page);

// softmax.hip
struct SoftmaxArgs {
    const float* x;
    float* y;
    int64_t ncols, nrows, n2, n3;
    int64_t xnb1, xnb2, xnb3, ynb1, ynb2, ynb3;  // bytes
    const void* mask;
    int mask_f16;
    int64_t mne2, mne3, mnb1, mnb2, mnb3;        // bytes
    float scale, max_bias;
};
int soft_max(const SoftmaxArgs& a, hipStream_t s);

// decoder_ops.hip
int swiglu(const float* a, int64_t anb1, const float* b, int64_t bnb1, float* y, int64_t ynb1, int64_t nc,
           int64_t nrows, hipStream_t s);
int rms_norm(const float* x, int64_t xnb1, float* y, int64_t ynb1, int64_t n, int64_t nrows, float eps,
             hipStream_t s);
// ROPE of q and k + SET_ROWS of k and v (F16 caches) in one launch
struct RopeKvArgs {
    const float* q;
    int64_t qnb1, qnb2;  // bytes per head, per token
    const float* k;
    int64_t knb1, knb2;
    const float* v;
    int64_t vnb1, vnb2;
    int64_t hd, Hq, Hkv, s;
    const int32_t* pos;
    float* qo;
    int64_t qonb1, qonb2;
    uint16_t* kc;
    int64_t kcnb1, kcnb2;  // bytes per cache row, per head
    uint16_t* vc;
    int64_t vcnb1, vcnb2;
    int64_t rows;
    const int64_t* idx;
    int32_t* n_bad;
    int n_dims, neox;
    float theta_scale, freq_scale, attn_factor;
};
int rope_kv(const RopeKvArgs& a, float freq_base, hipStream_t s);
int rope_cache(const int32_t* pos, int64_t n, int n_dims, float freq_base, float freq_scale, float attn_factor,
               float* y, int64_t ynb1, hipStream_t s);
int rope(const float* x, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, int64_t xnb1, int64_t xnb2, int64_t xnb3,
         const int32_t* pos, float* y, int64_t ynb1, int64_t ynb2, int64_t ynb3, int n_dims, int neox, float freq_base,
         float freq_scale, float attn_factor, hipStream_t s);
int add(const float* a, const int64_t* ane, const int64_t* anb, const float* b, const int64_t* bne,
        const int64_t* bnb, float* y, const int64_t* ynb, hipStream_t s);
int get_rows(const uint8_t* a, int atype, int64_t ne0, int64_t anb1, int64_t arows, const void* idx, int idx64,
             int64_t n, float* y, int64_t ynb1, hipStream_t s);
int argmax(const float* x, int64_t xnb1, int64_t n, int64_t nrows, int32_t* out, hipStream_t s);

// kv_step.hip
int kv_step_inputs(const int32_t* pos_dev, int64_t s, int32_t* pos_ids, int64_t* kv_idx, uint16_t* mask,
                   int64_t n_kv, int64_t mask_stride, hipStream_t st);
int kv_advance(int32_t* pos_dev, int64_t s, hipStream_t st);
int paged_step_inputs(const int32_t* pos, int64_t B, const int32_t* table, int64_t tstride, int log2p,
                      int64_t trash_row, int64_t* kv_idx, int32_t* seq_len, hipStream_t st);
int paged_advance(int32_t* pos, const int32_t* active, int64_t B, hipStream_t st);
int kv_pages_copy(uint8_t* pool, int64_t pnb1, int64_t pnb2, int64_t prows, uint8_t* cache, int64_t cnb1, int64_t cnb2,
                  const int32_t* pages, int64_t n_pages, int log2p, int64_t r0, int64_t r1, int64_t H,
                  int64_t row_bytes, int to_pool, hipStream_t st);


}  // namespace gq
