/*
 * gq_oracle — CPU restatement of the reference's quantized hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker. The product
 * path (ggmlc_amd/, libgq.so) never links, loads or calls it.
 *
 * Every function restates one piece of ggml 0.20.2 as vendored by ggmlc
 * (reference tree: third_party/ggml) or of ggmlc itself; the citation is on
 * each declaration. How each one is pinned (golden vectors from the compiled
 * reference, closed forms, brute force) is listed in tests/test_oracle.py.
 */
#ifndef GQ_ORACLE_H
#define GQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 <-> binary32, round to nearest even (F16C semantics used by
 * ggml_cpu_fp32_to_fp16, ggml-cpu/ggml-cpu.c:3444-3474; scalar form ggml-impl.h:407-431). */
uint16_t or_fp32_to_fp16(float f);
float or_fp16_to_fp32(uint16_t h);
void or_fp32_to_fp16_row(const float* x, uint16_t* y, int64_t n);

/* x86 runtime activation quantizer: ggml-cpu/arch/x86/quants.c:302-398.
 * amax = max|x|; d = fp16(amax/127.f); id = amax ? 127.f/amax : 0; q = RNE(x*id). */
void or_quantize_row_q8_0(const float* x, void* y, int64_t k);

/* ggml scalar reference quantizer: ggml-quants.c:276-299 (q = roundf(x/d), half away). */
void or_quantize_row_q8_0_ref(const float* x, void* y, int64_t k);

/* ggmlc's Python weight quantizers (python/ggmlc/quantization/quantize.py:10-25, 65-107),
 * numpy float32 semantics. These produce the .gguf weight bytes. */
void or_quantize_q8_0_py(const float* x, void* y, int64_t n);
void or_quantize_q4_0_py(const float* x, void* y, int64_t n);

/* Dequantizers: ggml-quants.c:459-476 (Q4_0), 553-566 (Q8_0). */
void or_dequantize_row_q8_0(const void* x, float* y, int64_t k);
void or_dequantize_row_q4_0(const void* x, float* y, int64_t k);

/* MUL_MAT with a quantized weight (ggml-cpu/ggml-cpu.c:1254-1452): src1 rows are
 * quantized with or_quantize_row_q8_0, each output is the block sum
 * sum_b d_w*d_a*isum_b (vec_dot_q{8,4}_0_q8_0, ggml-cpu/quants.c:225-256, 451-479).
 * W: N rows of K elements (type 8 = Q8_0, 2 = Q4_0), X: M rows of K fp32,
 * Y: M rows of N fp32. The block sums are accumulated in double; the reference
 * accumulates in float, so parity against it is a tolerance, not bit-exact.
 * n_threads > 1 splits rows of N across pthreads (same result). */
int or_mul_mat(int wtype, const void* w, int64_t K, int64_t N, const float* x, int64_t M,
               float* y, int n_threads);

/* Same, with X already quantized (M rows of K/32 Q8_0 blocks). */
int or_mul_mat_q8act(int wtype, const void* w, int64_t K, int64_t N, const void* xq, int64_t M,
                     float* y, int n_threads);

/* SET_ROWS F32 -> F16 (ggml-cpu/ops.cpp:5156-5259): for i < s and every (h, b):
 * dst[:, idx[i], h, b] = fp16_rne(src[:, i, h, b]). dst [hd, max_ctx, H, B], src [hd, s, H, B].
 * Returns -1 (and writes nothing) if any idx is outside [0, max_ctx), like the
 * reference's GGML_ASSERT. */
int or_set_rows_f32_f16(uint16_t* dst, int64_t hd, int64_t max_ctx, int64_t H, int64_t B,
                        const float* src, int64_t s, const int64_t* idx);

/* FLASH_ATTN_EXT, F16 K/V (ggml-cpu/ops.cpp:8532-8768 one_chunk and the split-KV
 * decode path :9179-9209 + reduce :9060-9128; tiled fp32 path :8770-9058 for s >= 64).
 *   q [hd, s, Hq] fp32, kc/vc caches [hd, max_ctx, Hkv] fp16 of which n_kv rows are
 *   read, mask [s][n_kv] fp16 or NULL, out [s][Hq][hd] fp32.
 * mode 0: the reference's arithmetic (fp16 Q, fp16 V accumulator for s < 64;
 *         n_split > 1 reproduces the split-KV chunking of an n_split-thread run).
 * mode 1: exact softmax(q.k*scale+mask).v in double (the mathematical target). */
int or_flash_attn_ext_f16(const float* q, int64_t hd, int64_t s, int64_t Hq,
                          const uint16_t* kc, const uint16_t* vc, int64_t max_ctx, int64_t Hkv,
                          int64_t n_kv, const uint16_t* mask, float scale, float* out, int mode,
                          int n_split);

/* SOFT_MAX f32 (ggml-cpu/ops.cpp:5519-5629): y = exp(x*scale + mask - max) / sum,
 * sum in double (ggml_float). x/y: nrows rows of ncols; mask fp16 [nrows][ncols] or NULL. */
int or_soft_max_f32(const float* x, int64_t ncols, int64_t nrows, const uint16_t* mask,
                    float scale, float* y);

/* ggmlc executor helpers: pad_kv_len (runtime/src/executor.cpp:58-64) and
 * fill_f16_causal_mask (executor.cpp:136-148, ATTN_MASK_MIN_FP16 = -32768). */
int64_t or_pad_kv_len(int64_t n_kv, int64_t max_ctx, int64_t n_pad);
void or_fill_causal_mask_f16(uint16_t* mask, int64_t pos, int64_t s_q, int64_t s_kv);

#ifdef __cplusplus
}
#endif
#endif
