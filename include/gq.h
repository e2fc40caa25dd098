/*
 * gq.h — C ABI of libgq.so, the MI355X (gfx950) implementation of ggmlc's
 * quantized execution hot path.
 *
 * Drop-in boundary: each entry point replaces one ggml operator that ggmlc's
 * executor emits on this path (reference citations on each declaration; paths
 * are relative to the reference checkout). Tensors cross the boundary as
 * gq_tensor, a plain descriptor with the same meaning as ggml_tensor's
 * data/type/ne/nb fields (third_party/ggml/include/ggml.h: ne = elements per
 * dimension, innermost first; nb = byte strides). Pointers are device pointers
 * owned by the caller; every call is asynchronous on the given HIP stream
 * (NULL = default stream); no call allocates device memory — scratch space is
 * passed in as a workspace whose size the matching *_workspace_size function
 * returns.
 *
 * Errors: every function returns GQ_OK (0) or a negative GQ_ERR_* code, and
 * gq_last_error() returns a thread-local message for the last failure. A
 * rejected call launches nothing, so the caller's state is untouched and the
 * library stays usable (the reference's contract, runtime/src/executor.cpp
 * :2411-2428 and tests/runtime/test_executor_cpu.cpp:106-119).
 */
#ifndef GQ_H
#define GQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GQ_ABI_VERSION 3

/* ggml type ids (third_party/ggml/include/ggml.h enum ggml_type; ggmlc
 * python/ggmlc/dialect/ggml/ops.py:39-108) */
enum gq_type {
    GQ_TYPE_F32 = 0,
    GQ_TYPE_F16 = 1,
    GQ_TYPE_Q4_0 = 2,
    GQ_TYPE_Q8_0 = 8,
    GQ_TYPE_I32 = 26,
    GQ_TYPE_I64 = 27,
};

enum gq_status {
    GQ_OK = 0,
    GQ_ERR_INVALID = -1,     /* bad shape / stride / type combination */
    GQ_ERR_UNSUPPORTED = -2, /* valid ggml call this build does not implement */
    GQ_ERR_WORKSPACE = -3,   /* workspace missing or too small */
    GQ_ERR_DEVICE = -4,      /* HIP runtime error (message has the HIP error string) */
};

/* opaque HIP stream (binary-compatible with hipStream_t) */
typedef struct ihipStream_t* gq_stream_t;

/* ggml_tensor's addressing fields. Shapes beyond the op's rank use ne = 1. */
typedef struct gq_tensor {
    void* data;
    int32_t type; /* enum gq_type */
    int32_t pad_;
    int64_t ne[4];
    size_t nb[4];
} gq_tensor;

/* ---- library ----------------------------------------------------------- */

int gq_abi_version(void);
const char* gq_last_error(void);
/* Checks that a gfx950 device is current and loads the kernels. */
int gq_init(void);

/* Process-wide switches. No counterpart in the reference (ggml has no such call):
 * they choose between launch plans that give the same bits, so a test or a
 * measurement can compare them. Unknown options or values return GQ_ERR_INVALID.
 *   GQ_OPT_ATTN_SEPARATE_MERGE (0 default / 1): decode attention merges its KV
 *   splits in a second launch instead of inside the decode kernel.
 *   GQ_OPT_GEMM_I8_RING (0 default / 1): the int8 path for 1..16 rows streams every
 *   product's weights and activation through its per-step register ring, also where a
 *   wave would otherwise request its whole tile at once, or take its activation from a
 *   copy staged in LDS once per workgroup. */
enum gq_option {
    GQ_OPT_ATTN_SEPARATE_MERGE = 1,
    GQ_OPT_GEMM_I8_RING = 2,
};
int gq_set_option(int option, int64_t value);

/* ---- quantize_row_q8_0 -------------------------------------------------- */

/* Replaces the x86 runtime quantizer the CPU backend runs on MUL_MAT's src1:
 * third_party/ggml/src/ggml-cpu/arch/x86/quants.c:302-398, reached through the
 * Q8_0 from_float trait (ggml-cpu/ggml-cpu.c:271-279) at ggml-cpu.c:1322-1357.
 * Same signature plus a stream: k floats (k % 32 == 0) -> k/32 block_q8_0.
 * Bit-exact: amax = max|x|; d = fp16_rne(amax/127); id = 127/amax (0 if amax
 * == 0); q = sat_int8(rne(x*id)). */
int gq_quantize_row_q8_0(const float* x, void* y, int64_t k, gq_stream_t stream);

/* Weight quantizers with ggmlc's compile-time semantics
 * (python/ggmlc/quantization/quantize.py:10-47 Q8_0, :65-107 Q4_0): n floats
 * (n % 32 == 0) -> n/32 blocks of `type` (GQ_TYPE_Q8_0 or GQ_TYPE_Q4_0). Used to
 * build device-resident weights with the exact bytes a .gguf would hold. */
int gq_quantize_weights(int type, const float* x, void* y, int64_t n, gq_stream_t stream);

/* ---- MUL_MAT ------------------------------------------------------------ */

/* Replaces ggml_mul_mat(a, b) (third_party/ggml/src/ggml.c:3278) as emitted by
 * the executor's MUL_MAT case (runtime/src/executor.cpp:2362-2447) for a
 * Q8_0/Q4_0 weight, computed as the CPU backend does
 * (ggml-cpu/ggml-cpu.c:1254-1452): src1 rows are quantized to Q8_0 with the
 * rule of gq_quantize_row_q8_0, then
 *     dst[n, m] = sum_b d_a[n,b] * d_x[m,b] * sum_{j<32} qa[n,b,j] * qx[m,b,j].
 *   a   : weight, type Q8_0 or Q4_0, ne = [K, N, 1, 1], contiguous
 *   b   : activation, F32, ne = [K, M, B2, B3], nb[0] = 4, rows contiguous
 *   dst : F32, ne = [N, M, B2, B3], nb[0] = 4
 * Small M runs an HBM-streaming GEMV over the native 34/18-byte blocks; large M
 * an LDS-tiled MFMA GEMM. Result: within 1e-3 max-abs-rel of the reference. */
size_t gq_mul_mat_workspace_size(const gq_tensor* a, const gq_tensor* b);
int gq_mul_mat(const gq_tensor* a, const gq_tensor* b, gq_tensor* dst, void* workspace,
               size_t workspace_bytes, gq_stream_t stream);

/* MUL_MAT fused with its neighbours in ggmlc's LLaMA graph (the node runs
 * executor.cpp:2034-2090 RMS_NORM, :2362-2447 MUL_MAT, GLU SWIGLU and ADD emit),
 * giving the bits of the unfused calls, applied in this order:
 *   b_add:    b := b + b_add first (gq_add(b, b_add): the residual ADD feeding the
 *             next RMS_NORM); the sum is also stored to b_sum when it is non-null
 *             (b_sum must not alias b or b_add)
 *   rms_norm: b's rows are RMS-normalized (gq_rms_norm with rms_eps)
 *   swiglu:   dst = SWIGLU(MUL_MAT(a, b)) over the two halves of a's rows
 *             (gq_swiglu of the [N, M] result): dst ne0 = N / 2
 *   bias:     MUL_MAT(a, b) + bias first, before the output-side fusions below (the
 *             MUL_MAT node's bias input, executor.cpp:2436-2445: ggml_add of an F32
 *             [N] row broadcast over the M rows); on both paths
 *   add:      dst = add + MUL_MAT(a, b) (gq_add); add may be dst itself
 *   rope_kv:  the rows of MUL_MAT(a, b) are a fused QKV projection,
 *             (n_head + 2 n_head_kv) heads of head_dim rows (q heads, k heads, v
 *             heads), and go through gq_rope_kv_store with the epilogue's
 *             arguments instead of being written: q rotated into q_out, k rotated
 *             and v copied into the caches at rows kv_idx (fp16). dst must be NULL.
 *             Modes 0 and 2; mode 2 needs n_dims == head_dim; head_dim a power of
 *             two (>= 4).
 * (swiglu, add and rope_kv exclude each other.) With M <= 4 activation rows (the
 * GEMV path) everything runs in one launch and needs no workspace. With M > 4 (the
 * GEMM path, K <= 16384) the input-side fusions run in the prologue that quantizes
 * the GEMM's activation (two launches), plus
 *   b_swiglu: the input is SWIGLU(b) of b's two halves (b ne0 = 2K: the gate|up
 *             product feeding the down projection), excluding rms_norm and b_add;
 * on the int8 path (5..16 rows, K % 256 == 0, 16-byte aligned weights) swiglu and
 * rope_kv also run as the product's epilogue (N % 16 == 0) and
 *   out_q8:   with swiglu, the SWIGLU rows are also written quantized for the next
 *             product (quantize_row_q8_0, the gq_q8_rows layout below for K = N / 2;
 *             N % 64 == 0); dst may then be NULL
 *   b_q8:     b's rows are already quantized in the gq_q8_rows layout (a producer's
 *             out_q8 or gq_flash_attn_paged_q8): no prologue; b gives the shape only,
 *             and the input-side fusions are excluded;
 *   int8:     the int8 path also for 1..4 rows (where the GEMV is the default), so a
 *             small batch can use the handoffs above;
 *   out_halves: plain products the int8 path takes in two halves of K
 *             (gq_mul_mat_fused_halves() == 1: at most 128 16-row tiles in 4 K parts,
 *             no bias, no output-side fusion) leave the two halves' sums to the
 *             consumer, one workgroup per half and tile: dst F32 [N, M, 2, 1] (b 2-d),
 *             slab h the sum over K's half h; the product is slab 0 + slab 1 in fp32,
 *             the bits of the call without out_halves. No counterpart in the
 *             reference: narrow products (the Qwen2.5-1.5B o and down projections) then
 *             stream on twice as many CUs;
 *   b_add_halves: b_add is such a pair, F32 [K, M, 2, 1]: the ADD adds slab 0 +
 *             slab 1 (GEMM path), so b + (slab 0 + slab 1) has the bits of the ADD of
 *             the unsplit product;
 * add with M > 4, the other output-side fusions off the int8 path, rope_kv shapes
 * outside the conditions above and b_swiglu on the GEMV path return
 * GQ_ERR_UNSUPPORTED and the caller runs those ops unfused. The GEMM path takes
 * workspace / workspace_bytes
 * (gq_mul_mat_fused_workspace_size). The ggml CUDA backend fuses the same neighbours
 * (ADD+RMS_NORM+MUL, MUL_MAT+GLU, MUL_MAT+ADD, ROPE+SET_ROWS) for the same reason:
 * these steps are launch-bound. */
typedef struct gq_rope_kv_epilogue {
    int32_t n_head, n_head_kv, head_dim;
    const gq_tensor* pos;   /* I32 [>= M] */
    int32_t n_dims, mode;
    float freq_base, freq_scale, attn_factor;
    const gq_tensor* kv_idx; /* I64 [M] */
    gq_tensor* q_out;        /* F32 [head_dim, n_head, M, 1] */
    gq_tensor* k_cache;      /* F16 [head_dim, rows, n_head_kv, 1] */
    gq_tensor* v_cache;
    int32_t* n_bad;          /* device int32 or NULL */
    const gq_tensor* rope_cache; /* gq_rope_cache of pos with the same n_dims/freq/attn
                                    arguments, F32 [n_dims, >= M], or NULL (computed
                                    in the launch: slower) */
} gq_rope_kv_epilogue;
typedef struct gq_mul_mat_fusion {
    int32_t rms_norm;
    float rms_eps;
    int32_t swiglu;
    const gq_tensor* add;
    const gq_tensor* b_add;
    gq_tensor* b_sum;
    const gq_rope_kv_epilogue* rope_kv;
    int32_t b_swiglu;        /* the input is SWIGLU of b's rows: b ne0 = 2K (GEMM path only) */
    void* workspace;         /* GEMM path: gq_mul_mat_fused_workspace_size bytes, 256-aligned */
    size_t workspace_bytes;
    const gq_tensor* bias;   /* F32 [N, 1, 1, 1] or NULL */
    void* out_q8;            /* int8 path with swiglu: the quantized SWIGLU rows, or NULL */
    const void* b_q8;        /* int8 path: b's rows already quantized, or NULL */
    int32_t int8;            /* 1: the int8 path for 1..16 rows, also 1..4 (GQ_ERR_UNSUPPORTED off it) */
    int32_t out_halves;      /* dst holds the sums of K's two halves (int8 path, see above) */
    int32_t b_add_halves;    /* b_add holds two slabs whose sum is added (GEMM path) */
} gq_mul_mat_fusion;
/* 1 when gq_mul_mat_fused(a, b, ., f) takes K in two halves, so f->out_halves may be
 * set (out_halves itself is ignored here), 0 when it does not, a negative GQ_ERR_*
 * when the call is invalid. */
int gq_mul_mat_fused_halves(const gq_tensor* a, const gq_tensor* b, const gq_mul_mat_fusion* f);
/* The quantized activation rows of the int8 path (up to 16 rows m of K values, K % 32
 * == 0; no counterpart in the reference, which quantizes src1 inside each MUL_MAT):
 * per quant block j of K, the 32 int8 quants of row m at byte (j * 16 + m) * 32, its
 * scale (fp32 value of the fp16 d) at K / 32 * 512 + (j * 16 + m) * 4 and its block sum
 * (int32) at K / 32 * 576 + (j * 16 + m) * 4 — the blocks of gq_quantize_row_q8_0
 * rearranged; gq_q8_rows_bytes(K) bytes, 16-byte aligned.
 * Rows past M are not written. */
size_t gq_q8_rows_bytes(int64_t K);
size_t gq_mul_mat_fused_workspace_size(const gq_tensor* a, const gq_tensor* b, const gq_mul_mat_fusion* f);
int gq_mul_mat_fused(const gq_tensor* a, const gq_tensor* b, gq_tensor* dst, const gq_mul_mat_fusion* f,
                     gq_stream_t stream);

/* ---- SET_ROWS ----------------------------------------------------------- */

/* Replaces ggml_set_rows(a, b, c) (ggml.c:3937-3962) with the CPU semantics of
 * ggml-cpu/ops.cpp:5156-5259 for an F16 destination and F32 source — the KV
 * cache write of runtime/src/executor.cpp:2181-2184:
 *     a[:, c[i, i2 % ne_c1, i3 % ne_c2], i2, i3] = fp16_rne(b[:, i, i2, i3])
 *   a : F16 cache ne = [hd, rows, H, B] (rows contiguous: nb[0] = 2); updated in place
 *   b : F32 ne = [hd, s, H, B], nb[0] = 4
 *   c : I64 (or I32) row indices ne = [s, ne_c1, ne_c2, 1]
 * Bit-exact. Indices outside [0, rows) are skipped and counted in *n_bad when
 * n_bad (a device int32) is non-NULL (the reference aborts on them). */
int gq_set_rows(gq_tensor* a, const gq_tensor* b, const gq_tensor* c, int32_t* n_bad,
                gq_stream_t stream);

/* ---- FLASH_ATTN_EXT ----------------------------------------------------- */

/* Replaces ggml_flash_attn_ext(q, k, v, mask, scale, max_bias, logit_softcap)
 * (ggml.c:5402-5437) as the executor emits it over the padded KV view
 * (runtime/src/executor.cpp:2143-2197): computes for each query row i and head h
 *     out[:, h, i] = softmax_j(scale * q[:, i, h] . k[:, j, h / (Hq/Hkv)] + mask[j, i]) v[:, j, ...]
 *   q    : F32 ne = [D, S, Hq, 1]
 *   k, v : F16 ne = [D, n_kv, Hkv, 1] (any row/head strides, nb[0] = 2)
 *   mask : F16 ne = [n_kv, >= S, 1, 1] or NULL
 *   dst  : F32 ne = [D, Hq, S, 1] contiguous (the op's permuted output)
 * D a multiple of 8 up to 256: the head dims ggmlc's executor sends to flash attention
 * (40, 64, 72, 80, 96, 112, 128, 192, 256; executor.cpp:2306-2309) and the ones it runs
 * through its soft_max fallback; 64 and 128 take the matrix-core prefill kernel, the
 * others the VALU kernels padded to 64, 128 or 256 dims (the padded dims read 0 and are
 * not stored). One query row with 2..16 query heads per kv head (head dim 64 or 128, no
 * ALiBi or softcap, 16-byte K/V rows, an 8-byte aligned mask and n_kv % 4 == 0 when a
 * mask is given) decodes on the matrix cores in 128-row splits. max_bias and
 * logit_softcap follow ops.cpp:8532-8768. Query rounding follows the CPU path taken for
 * that S (fp16 for S < 64, fp32 for S >= 64); accumulation is fp32. Decode launches
 * (few query vectors per kv head) merge their KV splits inside the kernel through
 * arrival counters that belong to the launch's stream (16 streams per process have
 * their own; launches on further streams merge in a second launch), so calls on
 * different streams may overlap; graphs captured on one stream must not be replayed
 * concurrently. */
size_t gq_flash_attn_ext_workspace_size(const gq_tensor* q, const gq_tensor* k);
int gq_flash_attn_ext(const gq_tensor* q, const gq_tensor* k, const gq_tensor* v,
                      const gq_tensor* mask, float scale, float max_bias, float logit_softcap,
                      gq_tensor* dst, void* workspace, size_t workspace_bytes,
                      gq_stream_t stream);

/* gq_flash_attn_ext without a workspace, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Same validation, kernels and bits as
 * gq_flash_attn_ext; the KV-split partials go to a static device array of
 * GQ_ATTN_SCRATCH_BYTES (16 MiB) that each device holds until the process ends
 * (its address is looked up by gq_init, or by the first call on the device). A
 * shape whose partials need more (gq_flash_attn_ext_workspace_size) returns
 * GQ_ERR_WORKSPACE before anything launches. Calls share the array, so two calls
 * that overlap on one device race: issue them on one stream. */
#define GQ_ATTN_SCRATCH_BYTES ((size_t)16 << 20)
int gq_flash_attn_ext_noalloc(const gq_tensor* q, const gq_tensor* k, const gq_tensor* v,
                              const gq_tensor* mask, float scale, float max_bias, float logit_softcap,
                              gq_tensor* dst, gq_stream_t stream);

/* Zeroes the arrival counters of the decode kernels' in-kernel split merge (every
 * stream's set on the current device; a fill kernel on `stream`, safe inside graph
 * capture). Every completed launch leaves them at zero; a caller whose decode attention
 * launch did not run to completion (an aborted graph, an error between capture and
 * replay) calls this on the device, with no decode attention in flight, before its next
 * decode attention. No counterpart in the reference. */
int gq_attn_reset_counters(gq_stream_t stream);

/* ---- SOFT_MAX ----------------------------------------------------------- */

/* Replaces ggml_soft_max_ext(a, mask, scale, max_bias) (ggml.c:4081-4105;
 * CPU ops.cpp:5519-5629): dst = softmax(a*scale + slope*mask) per row.
 *   a, dst : F32 ne = [ncols, nrows, n2, n3], rows contiguous
 *   mask   : F16 or F32 ne = [ncols, >= nrows, ...] (broadcast over dims 2,3) or NULL */
int gq_soft_max(const gq_tensor* a, const gq_tensor* mask, float scale, float max_bias,
                gq_tensor* dst, gq_stream_t stream);

/* ---- decoder ops around the quantized path -------------------------------
 * The remaining nodes of a LLaMA-style layer as the executor emits them
 * (runtime/src/executor.cpp:2034-2090, 2355-2357, 2742-2756). F32 activations;
 * rows (dim 0) contiguous; all other dims may be strided. */

/* ggml_swiglu(a) / ggml_swiglu_swapped(a) (ggml.c:3048-3058; CPU ops.cpp:3246):
 * per row, y = silu(a[0:nc]) * a[nc:2nc] (halves exchanged when swapped). With
 * b != NULL it is ggml_swiglu_split(a, b): y = silu(a) * b. dst ne = [nc, rows]. */
int gq_swiglu(const gq_tensor* a, const gq_tensor* b, gq_tensor* dst, int swapped, gq_stream_t stream);

/* ggml_rms_norm(a, eps) (CPU ops.cpp rms_norm_f32): y = x / sqrt(mean(x^2) + eps) per row. */
int gq_rms_norm(const gq_tensor* a, float eps, gq_tensor* dst, gq_stream_t stream);

/* ggml_rope_ext(a, pos, NULL, n_dims, mode, n_ctx_orig, freq_base, freq_scale,
 * ext_factor, attn_factor, beta_fast, beta_slow) (ggml.c; CPU ops.cpp:5886-6120)
 * for mode 0 (NORMAL) and 2 (NEOX) with ext_factor == 0 (no YaRN ramp; n_ctx_orig
 * and the betas only enter through it). a F32 ne = [hd, heads, seq, B],
 * pos I32 [seq]. */
int gq_rope_ext(const gq_tensor* a, const gq_tensor* pos, int n_dims, int mode, int n_ctx_orig, float freq_base,
                float freq_scale, float ext_factor, float attn_factor, float beta_fast, float beta_slow,
                gq_tensor* dst, gq_stream_t stream);

/* ROPE of q and k plus SET_ROWS of k and v: the node sequence between the fused QKV
 * projection and FLASH_ATTN_EXT (executor.cpp:2034-2090 rope, :2181-2184 set_rows) in
 * one launch, bit-identical to
 *   q_out = gq_rope_ext(q); k' = gq_rope_ext(k);
 *   gq_set_rows(k_cache, permute(k', 0, 2, 1, 3), kv_idx); gq_set_rows(v_cache, permute(v, ...), kv_idx)
 *   q, k, v  F32 [hd, H, s, 1] (rows contiguous; e.g. views of the QKV output)
 *   pos      I32 [>= s]; kv_idx I64 [s]
 *   q_out    F32 [hd, Hq, s, 1]
 *   k_cache, v_cache F16 [hd, rows, Hkv, 1]
 * Modes 0 and 2, ext_factor 0. Out-of-range indices are skipped and counted (per
 * token and head) in *n_bad when it is non-null. */
int gq_rope_kv_store(const gq_tensor* q, const gq_tensor* k, const gq_tensor* v, const gq_tensor* pos, int n_dims,
                     int mode, float freq_base, float freq_scale, float attn_factor, const gq_tensor* kv_idx,
                     gq_tensor* q_out, gq_tensor* k_cache, gq_tensor* v_cache, int32_t* n_bad, gq_stream_t stream);

/* The ROPE cache of ggml_rope_cache_init (CPU ops.cpp:5910-5925) for modes 0/2 with
 * ext_factor 0: dst[2j, i], dst[2j+1, i] = cos, sin(pos[i] * theta_scale^j * freq_scale)
 * * attn_factor for j < n_dims/2, theta_scale = freq_base^(-2/n_dims), built by repeated
 * multiplication as there. pos I32 [n]; dst F32 [n_dims, n], rows contiguous. Every
 * layer's rope at these positions uses the same table, so a decode step computes it
 * once for the QKV epilogue (gq_rope_kv_epilogue.rope_cache); same bits as in-kernel. */
int gq_rope_cache(const gq_tensor* pos, int n_dims, float freq_base, float freq_scale, float attn_factor,
                  gq_tensor* dst, gq_stream_t stream);

/* ggml_add(a, b) with b repeated over a (ggml_can_repeat). */
int gq_add(const gq_tensor* a, const gq_tensor* b, gq_tensor* dst, gq_stream_t stream);

/* ggml_get_rows(a, b): a (Q8_0, Q4_0, F16 or F32) ne = [n_embd, rows], b I32/I64 [n]
 * -> dst F32 [n_embd, n]. Out-of-range ids give zero rows. */
int gq_get_rows(const gq_tensor* a, const gq_tensor* b, gq_tensor* dst, gq_stream_t stream);

/* ggml_argmax(a): first index of the row maximum, dst I32 [rows]. */
int gq_argmax(const gq_tensor* a, gq_tensor* dst, gq_stream_t stream);

/* ---- persistent-KV step inputs --------------------------------------------
 * The per-step inputs ggmlc's executor writes on the host before each run —
 * set_decode_pos / set_chunk_pos (runtime/src/executor.cpp:1181-1393) and
 * fill_f16_causal_mask (:136-148) — computed on the device from a position that
 * lives in device memory (*pos, int32), so a captured step graph replays without
 * host work:
 *   pos_ids[i] = kv_idx[i] = *pos + i for i < s   (either may be NULL)
 *   mask F16 [n_kv, >= s]: mask[j, i] = 0 if j <= *pos + i else -32768 (NULL: none).
 * gq_kv_advance adds s to *pos (the last node of a decode-step graph). */
int gq_kv_step_inputs(const int32_t* pos, int64_t s, int32_t* pos_ids, int64_t* kv_idx, gq_tensor* mask,
                      gq_stream_t stream);
int gq_kv_advance(int32_t* pos, int64_t s, gq_stream_t stream);

/* ---- paged KV: batched decode over a page pool ---------------------------------
 * ggmlc's paged KV (runtime/src/executor.cpp:634-920, VMM windows of
 * vmm_pool.cu) gives every batch slot its own KV rows; the continuous-batching
 * scheduler (batch_scheduler.cpp:130-405) then decodes all active slots in one
 * graph. Here a pool holds pages of `page_size` rows (a power of two >= 64,
 * 128 for D = 64) per layer, F16 [D, rows, Hkv, 1]; a page table I32
 * [max_pages, B] lists each sequence's pages in order, so logical row r of
 * sequence b is pool row table[b][r / P] * P + r % P. Pages are shared between
 * sequences by listing them in several rows of the table (prefix caching). */

/* Batched decode attention: ggml_flash_attn_ext (ggml.c:5402-5437; CPU
 * ops.cpp:9130-9264) of every sequence's one new token over that sequence's own
 * rows, each with its own length (the reference shares one position across the
 * batch, batch_scheduler.cpp:302-321; here every sequence keeps its own):
 *   out[:, h, b] = softmax_{j < seq_len[b]}(scale * q[:, b, h] . k_b[:, j, h / G]) v_b[:, j, ...]
 *   q        : F32 [D, B, Hq, 1]  (row b = sequence b; the query is rounded to fp16
 *              like the CPU decode path)
 *   k/v_pool : F16 [D, rows, Hkv, 1], one head of a pool below 2 GiB
 *   page_table, seq_len : device I32 (a negative page id reads nothing)
 *   max_len  : an upper bound of every seq_len[b] (sizes the launch)
 *   dst      : F32 [D, Hq, B] contiguous.  D in {64, 128}, Hq / Hkv <= 8 (<= 16 when
 *              page_size is a multiple of 128; groups of 2-16 run on the matrix cores).
 * Equal to the reference's decode step of sequence b with the causal mask of its
 * position (columns past it weigh exactly 0). Its in-kernel split merge counts
 * arrivals per stream, like gq_flash_attn_ext's. */
size_t gq_flash_attn_paged_workspace_size(const gq_tensor* q, const gq_tensor* k_pool, int64_t max_len,
                                          int64_t page_size);
int gq_flash_attn_paged(const gq_tensor* q, const gq_tensor* k_pool, const gq_tensor* v_pool,
                        const gq_tensor* page_table, const gq_tensor* seq_len, int64_t page_size, int64_t max_len,
                        float scale, gq_tensor* dst, void* workspace, size_t workspace_bytes, gq_stream_t stream);
/* gq_flash_attn_paged that also writes dst's B rows (Hq * D values each) quantized for
 * the output projection into out_q8 (the gq_q8_rows layout, K = Hq * D): the prologue of
 * that projection's MUL_MAT done by the split merge, so the projection can take them
 * through gq_mul_mat_fusion.b_q8. No counterpart in the reference (one fewer launch per
 * layer for the batched decode). B <= 16, 2..16 query heads per kv head (the
 * matrix-core kernel), max_len > 128 (a split merge runs). */
int gq_flash_attn_paged_q8(const gq_tensor* q, const gq_tensor* k_pool, const gq_tensor* v_pool,
                           const gq_tensor* page_table, const gq_tensor* seq_len, int64_t page_size, int64_t max_len,
                           float scale, gq_tensor* dst, void* out_q8, void* workspace, size_t workspace_bytes,
                           gq_stream_t stream);

/* Per-slot inputs of a batched decode step from device-resident positions pos[B]
 * (the per-slot set_decode_pos of executor.cpp:1181-1276):
 *   kv_idx[b] = the pool row position pos[b] is written to (trash_row when its page
 *   is missing), seq_len[b] = pos[b] + 1 (0 when missing; seq_len may be NULL).
 * gq_paged_advance adds 1 to pos[b] where active[b] != 0 (active NULL: every slot). */
int gq_paged_step_inputs(const int32_t* pos, int64_t B, const gq_tensor* page_table, int64_t page_size,
                         int64_t trash_row, int64_t* kv_idx, int32_t* seq_len, gq_stream_t stream);
int gq_paged_advance(int32_t* pos, const int32_t* active, int64_t B, gq_stream_t stream);

/* Rows [r0, r1) of one sequence between a contiguous F16 cache [D, ctx, H, 1] (row r)
 * and its pages in a pool [D, rows, H, 1] (pages: device I32 [n_pages] page ids):
 * to_pool = 1 stores computed rows into the pages, 0 loads shared pages into the
 * cache — what mapping existing pages into a slot's window does in the reference
 * (paged_kv_map_existing_pages / paged_kv_extract_page_handles, executor.cpp:838-920). */
int gq_kv_pages_copy(gq_tensor* pool, gq_tensor* cache, const int32_t* pages, int64_t n_pages, int64_t page_size,
                     int64_t r0, int64_t r1, int to_pool, gq_stream_t stream);

/* ---- executor handle --------------------------------------------------------
 * ggmlc's ModelExecutor (runtime/include/ggmlc/executor.h:25-289; the surface its
 * Python binding exposes, runtime/bindings/python_bindings.cpp:137-216) for the graphs
 * this library executes: a ggmlc .gguf (GGUF v3 whose `ggmlc.graph_spec` JSON is the
 * execution graph, runtime/src/loader.cpp:77-443) whose graph is the LLaMA-family
 * decoder layout ggmlc's compiler emits (embedding GET_ROWS; per layer RMS_NORM -> QKV
 * MUL_MAT (fused with three VIEWs, or three products; optional F32 bias inputs) ->
 * RESHAPE -> NEOX ROPE (q, k) -> PERMUTE -> FLASH_ATTN_EXT -> RESHAPE -> MUL_MAT -> ADD,
 * RMS_NORM -> gate|up MUL_MAT -> GLU SWIGLU -> MUL_MAT -> ADD; RMS_NORM -> head MUL_MAT).
 * A graph outside it is rejected with GQ_ERR_UNSUPPORTED naming the first node that
 * does not fit. Weights are the file's bytes, uploaded once; each step runs the
 * decoder on this library's kernels, replayed from one HIP graph per (s, n_kv, output
 * rows) bucket after that bucket's first run. The handle owns its device memory and a
 * stream of default priority. One handle per thread (not re-entrant), as in the reference.
 *
 *   device: "auto", "gpu", "cuda" (device 0), "gpu:N", "cuda:N"; anything else, or no
 *   visible GPU, is an error (this runtime has no CPU path).
 *   symbols: "s" (tokens this step, required) and "pos" (position of the first; default
 *   the handle's running position with a KV cache, else 0).
 *   The input is the graph's token-id tensor (I32 or I64, s values); the output its
 *   logits, F32 [n_vocab, s] (rows = tokens), or [n_vocab, 1] with logits_last_only
 *   (executor.cpp:2396-2410). Without init_kv_cache each run is a whole sequence from
 *   position 0 in a scratch cache. n_kv follows pad_kv_len (executor.cpp:58-64) with the
 *   pad GGMLC_KV_PAD gives when the cache is initialised (default 256, executor.cpp:501-503). */
typedef struct gq_exec gq_exec;
/* ModelExecutor::get_available_devices (executor.cpp:184): JSON list of "cuda:N" for the
 * visible GPUs (no CPU entry: this runtime has no CPU path). */
int gq_exec_available_devices(char* buf, size_t buf_len, size_t* needed);
int gq_exec_create(const void* gguf_bytes, size_t len, const char* device, gq_exec** out);
void gq_exec_free(gq_exec* h);
/* JSON: name, device, inputs, outputs, parameters, symbol_table, names {id: name},
 * embed / lm_head / layers (the matched weights), config (hyper-parameters). The call
 * writes at most buf_len bytes (NUL-terminated) and the full size + 1 to *needed. */
int gq_exec_describe(gq_exec* h, char* buf, size_t buf_len, size_t* needed);
/* The same description of a model without a device (parse and match only). */
int gq_exec_inspect(const void* gguf_bytes, size_t len, char* buf, size_t buf_len, size_t* needed);
int gq_exec_prepare(gq_exec* h, const char* const* sym_names, const int64_t* sym_values, int64_t n_syms);
int gq_exec_set_input(gq_exec* h, uint32_t tensor_id, const void* data, size_t bytes);
int gq_exec_set_input_by_name(gq_exec* h, const char* name, const void* data, size_t bytes);
/* Runs the prepared step synchronously; the output is then held on the host. */
int gq_exec_run(gq_exec* h);
int gq_exec_synchronize(gq_exec* h);
int gq_exec_get_tensor_shape(gq_exec* h, uint32_t tensor_id, int64_t ne[4]);
/* Copies the output's bytes (F32, rows of n_vocab) to dst when dst_bytes suffices;
 * *written (if non-NULL) receives the output's size either way. */
int gq_exec_get_output(gq_exec* h, uint32_t tensor_id, void* dst, size_t dst_bytes, size_t* written);
int gq_exec_init_kv_cache(gq_exec* h, int64_t max_ctx);
int gq_exec_reset_kv_cache(gq_exec* h);
int gq_exec_has_kv_cache(gq_exec* h);
int gq_exec_set_logits_last_only(gq_exec* h, int enable);
int gq_exec_logits_last_only(gq_exec* h);
/* HIP graph replay of the step buckets (on by default; the reference's
 * set_enable_cuda_graph). */
int gq_exec_set_enable_graphs(gq_exec* h, int enable);
/* The handle's running position (tokens written to the KV cache), -1 for NULL. */
int64_t gq_exec_position(gq_exec* h);

/* ---- paged KV cache and batched decode (ModelExecutor::init_paged_kv_cache,
 * paged_kv_*, get_paged_active_vram_bytes, set/get_tokens_per_page: executor.h:73-93,
 * executor.cpp:634-920) ------------------------------------------------------------
 * Per layer one K and one V page pool sized for max_batch slots of max_ctx rows; a page
 * holds tokens_per_page rows of every layer (default 128; a power of two >= 64, >= 128
 * for head_dim 64, set before init) and is named by one int32 id for all layers (the
 * reference's per-layer VMM handles, executor.cpp:838-920). Pages are reference counted:
 * a slot holds one reference per page it lists (ensure_tokens allocates, map_existing_pages
 * shares, free_slot releases); a caller that keeps pages beyond their slot (a prefix cache)
 * retains them (gq_exec_paged_page_retain) and releases them later.
 * With the paged cache on, gq_exec_prepare takes the reference scheduler's symbols
 * (batch_scheduler.cpp:190-194, 318-321):
 *   {s, slot[, pos][, b = 1]}: a prompt step of that slot, s tokens at pos (default: the
 *     slot's position), computed on the contiguous cache (its graphs) and stored into the
 *     slot's pages; the slot then continues at pos + s. Output: the logits of the step.
 *   {b, s = 1[, pos]}: one decode token for every slot of [0, b) (input: b token ids),
 *     each slot at its own position (the reference runs the batch at the largest, pos;
 *     here pos only has to cover every allocated slot's position), the slots' positions
 *     then advance by one. Slots without pages write a trash page and attend to nothing.
 *     Output: F32 [n_vocab, b], row i the logits of slot i. One HIP graph per (b, context
 *     bucket of 512 rows); 2..16 rows run the int8 product chain.
 * Every slot must hold rows for the positions it runs (paged_kv_ensure_tokens). */
int gq_exec_set_tokens_per_page(gq_exec* h, int64_t tokens_per_page);
int64_t gq_exec_get_tokens_per_page(gq_exec* h);
/* Allocates the pools (and the contiguous cache of max_ctx rows when init_kv_cache has
 * not run); a second call changes nothing (executor.cpp:635). */
int gq_exec_init_paged_kv_cache(gq_exec* h, int64_t max_batch, int64_t max_ctx);
int gq_exec_is_paged_kv_cache_enabled(gq_exec* h);
/* Marks the slot in use at position 0 with no pages (an allocated slot is freed first). */
int gq_exec_paged_kv_alloc_slot(gq_exec* h, int64_t slot);
int gq_exec_paged_kv_free_slot(gq_exec* h, int64_t slot);
int gq_exec_is_paged_slot_allocated(gq_exec* h, int64_t slot);
/* Gives the slot pages for rows [0, total_tokens); GQ_ERR_WORKSPACE when the pool is out
 * of free pages. */
int gq_exec_paged_kv_ensure_tokens(gq_exec* h, int64_t slot, int64_t total_tokens);
/* Appends existing pages (ids from gq_exec_paged_kv_extract_page) as the slot's pages
 * start_page.. (start_page must equal the slot's page count), one reference each. */
int gq_exec_paged_kv_map_existing_pages(gq_exec* h, int64_t slot, int64_t start_page, const int32_t* pages,
                                        int64_t n_pages);
/* The id of the slot's page page_idx (paged_kv_extract_page_handles). */
int gq_exec_paged_kv_extract_page(gq_exec* h, int64_t slot, int64_t page_idx, int32_t* page);
int gq_exec_paged_page_retain(gq_exec* h, int32_t page);
int gq_exec_paged_page_release(gq_exec* h, int32_t page);
/* Device bytes of the pages in use (every layer, K and V). */
size_t gq_exec_get_paged_active_vram_bytes(gq_exec* h);
/* A slot's position (its next row), and setting it (rewinding a slot). No counterpart in
 * the reference, whose scheduler tracks positions outside the executor. */
int gq_exec_paged_slot_position(gq_exec* h, int64_t slot, int64_t* pos);
int gq_exec_paged_set_slot_position(gq_exec* h, int64_t slot, int64_t pos);

/* ---- profiling (ModelExecutor::set_enable_profile, reset_profile, get_profile,
 * runtime_graph_summary, runtime_mul_mat_shape_summary: executor.h:101-118,
 * executor.cpp:3184-3459) -----------------------------------------------------------
 * With profiling on, prepare and run add their host wall time (run: the whole step,
 * graph replay and the logits' download included). The set_*_pos and mask fields stay 0:
 * positions, row indices and the causal mask are computed on the device inside the step. */
typedef struct gq_exec_profile {
    double prepare_ms, set_decode_pos_ms, set_chunk_pos_ms, mask_fill_ms, run_ms;
    int32_t n_prepare, n_set_decode_pos, n_set_chunk_pos, n_run;
} gq_exec_profile;
int gq_exec_set_enable_profile(gq_exec* h, int enable);
int gq_exec_reset_profile(gq_exec* h);
int gq_exec_get_profile(gq_exec* h, gq_exec_profile* out);
/* JSON of the last issued step: n_nodes (launches), n_kernel_nodes (the replayed graph's
 * nodes, else the launches), n_mul_mat, n_flash_attn, n_set_rows (launches that contain
 * them: fused launches count once each), kv_n_pad, graphs_captured, last_run_replayed,
 * paged_kv and ops {launch: count} (a launch named by the ops it runs, e.g.
 * "RMS_NORM+ADD+MUL_MAT+ROPE+SET_ROWS"). Same output convention as gq_exec_describe. */
int gq_exec_runtime_graph_summary(gq_exec* h, char* buf, size_t buf_len, size_t* needed);
/* JSON {mul_mat: [{n, shape}], flash_attn: [{n, shape}]}: the products' (type, K, N, M)
 * and the attention launches' shapes of the last issued step, most frequent first. */
int gq_exec_runtime_mul_mat_shape_summary(gq_exec* h, char* buf, size_t buf_len, size_t* needed);

#ifdef __cplusplus
}
#endif
#endif /* GQ_H */
