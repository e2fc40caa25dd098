/*
 * gq_oracle.c — CPU restatement of the reference's quantized hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see gq_oracle.h). Plain C, scalar, written from the
 * semantics of the cited reference functions; it is the checker for the HIP
 * path and is pinned itself against the compiled reference (oracle/_ref) and
 * against closed forms in tests/test_oracle.py.
 *
 * Built with -ffp-contract=off so that a*b+c is never fused unless fmaf() is
 * written explicitly (the reference's AVX2 code uses explicit FMA in exactly the
 * places where fmaf appears below).
 */
#include "gq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define QK 32

/* ---------------------------------------------------------------- fp16 --- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* binary32 -> binary16, round to nearest, ties to even; NaN stays NaN (quiet),
 * overflow -> inf, tiny values -> subnormal/zero with correct rounding. */
uint16_t or_fp32_to_fp16(float f) {
    const uint32_t u = f2u(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t au = u & 0x7fffffffu;
    if (au >= 0x7f800000u) { /* inf or NaN */
        if (au == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((au >> 13) & 0x3ffu);
    }
    const int32_t e = (int32_t)(au >> 23) - 127; /* unbiased exponent */
    if (e > 15) return sign | 0x7c00u;            /* rounds to inf */
    uint32_t mant = (au & 0x7fffffu) | (e > -127 ? 0x800000u : 0u);
    /* value = mant * 2^(e-23) (normal) ; target ulp for normals is 2^(e-10),
     * for subnormals 2^-24. Shift = number of bits dropped. */
    int32_t shift;
    uint32_t base_exp; /* biased half exponent applied after rounding */
    if (e >= -14) { shift = 13; base_exp = (uint32_t)(e + 15); }
    else {
        shift = 13 + (-14 - e);
        base_exp = 0;
        if (e == -127) shift = 13 + (-14 - (-126)); /* float subnormal input */
        if (shift > 24 + 1) return sign;              /* < half of smallest subnormal */
    }
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    if (base_exp == 0) {
        /* subnormal result; q may have rounded up into the normal range (q == 0x400) */
        return sign | (uint16_t)q;
    }
    /* q holds the implicit bit at 0x400; rounding may carry to 0x800 */
    uint32_t h = (base_exp << 10) + (q - 0x400u);
    if (q >= 0x800u) h = ((base_exp + 1u) << 10);
    if (h >= 0x7c00u) return sign | 0x7c00u;
    return sign | (uint16_t)h;
}

float or_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return u2f(sign);
        /* subnormal: m * 2^-24, exact in float */
        const float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void or_fp32_to_fp16_row(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_fp32_to_fp16(x[i]);
}

/* ----------------------------------------------------------- quantizers --- */

typedef struct { uint16_t d; int8_t qs[QK]; } blk_q8;      /* ggml-common.h:251-256 */
typedef struct { uint16_t d; uint8_t qs[QK / 2]; } blk_q4; /* ggml-common.h:194-199 */

/* arch/x86/quants.c:302-398 (AVX2 branch). */
void or_quantize_row_q8_0(const float* x, void* vy, int64_t k) {
    unsigned char* y = (unsigned char*)vy;
    const int64_t nb = k / QK;
    for (int64_t i = 0; i < nb; ++i) {
        const float* xb = x + i * QK;
        float amax = 0.0f;
        for (int j = 0; j < QK; ++j) {
            const float a = fabsf(xb[j]);
            amax = a > amax ? a : amax;
        }
        const float d = amax / 127.f;
        const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
        const uint16_t dh = or_fp32_to_fp16(d);
        memcpy(y + i * 34, &dh, 2);
        for (int j = 0; j < QK; ++j) {
            float v = rintf(xb[j] * id); /* _mm256_round_ps(_MM_ROUND_NEAREST) */
            int32_t iv = (int32_t)v;
            if (iv > 127) iv = 127;       /* packs_epi32 / packs_epi16 saturation */
            if (iv < -128) iv = -128;
            y[i * 34 + 2 + j] = (unsigned char)(int8_t)iv;
        }
    }
}

/* ggml-quants.c:276-299 */
void or_quantize_row_q8_0_ref(const float* x, void* vy, int64_t k) {
    unsigned char* y = (unsigned char*)vy;
    const int64_t nb = k / QK;
    for (int64_t i = 0; i < nb; ++i) {
        const float* xb = x + i * QK;
        float amax = 0.0f;
        for (int j = 0; j < QK; ++j) {
            const float a = fabsf(xb[j]);
            amax = amax > a ? amax : a;
        }
        const float d = amax / ((1 << 7) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        const uint16_t dh = or_fp32_to_fp16(d);
        memcpy(y + i * 34, &dh, 2);
        for (int j = 0; j < QK; ++j) {
            const float x0 = xb[j] * id;
            y[i * 34 + 2 + j] = (unsigned char)(int8_t)roundf(x0);
        }
    }
}

/* quantize.py:10-25 — numpy float32: scale = amax/127; inv = f32(1/scale);
 * q = clip(RNE(x*inv), -128, 127); d = fp16(scale). n is padded to a block with zeros. */
void or_quantize_q8_0_py(const float* x, void* vy, int64_t n) {
    unsigned char* y = (unsigned char*)vy;
    const int64_t nb = (n + QK - 1) / QK;
    for (int64_t i = 0; i < nb; ++i) {
        float xb[QK];
        for (int j = 0; j < QK; ++j) xb[j] = (i * QK + j < n) ? x[i * QK + j] : 0.0f;
        float amax = 0.0f;
        for (int j = 0; j < QK; ++j) {
            const float a = fabsf(xb[j]);
            amax = a > amax ? a : amax;
        }
        const float scale = amax > 0.0f ? amax / 127.0f : 0.0f;
        const float safe = scale != 0.0f ? scale : 1.0f;
        const float inv = 1.0f / safe;
        const uint16_t dh = or_fp32_to_fp16(scale);
        memcpy(y + i * 34, &dh, 2);
        for (int j = 0; j < QK; ++j) {
            float v = rintf(xb[j] * inv);
            if (v < -128.0f) v = -128.0f;
            if (v > 127.0f) v = 127.0f;
            y[i * 34 + 2 + j] = (unsigned char)(int8_t)(int32_t)v;
        }
    }
}

/* quantize.py:65-107 — signed max (first index of max |x|), scale = smax / -8,
 * q = clip(RNE(x / scale) + 8, 0, 15) (8 when scale == 0); low nibbles hold
 * elements 0..15, high nibbles 16..31. */
void or_quantize_q4_0_py(const float* x, void* vy, int64_t n) {
    unsigned char* y = (unsigned char*)vy;
    const int64_t nb = (n + QK - 1) / QK;
    for (int64_t i = 0; i < nb; ++i) {
        float xb[QK];
        for (int j = 0; j < QK; ++j) xb[j] = (i * QK + j < n) ? x[i * QK + j] : 0.0f;
        int imax = 0;
        float amax = fabsf(xb[0]);
        for (int j = 1; j < QK; ++j) {
            const float a = fabsf(xb[j]);
            if (a > amax) { amax = a; imax = j; }
        }
        const float smax = xb[imax];
        const float scale = smax != 0.0f ? smax / -8.0f : 0.0f;
        const float safe = scale != 0.0f ? scale : 1.0f;
        const uint16_t dh = or_fp32_to_fp16(scale);
        memcpy(y + i * 18, &dh, 2);
        uint8_t q[QK];
        for (int j = 0; j < QK; ++j) {
            if (scale == 0.0f) { q[j] = 8; continue; }
            float v = rintf(xb[j] / safe) + 8.0f;
            if (v < 0.0f) v = 0.0f;
            if (v > 15.0f) v = 15.0f;
            q[j] = (uint8_t)v;
        }
        for (int j = 0; j < QK / 2; ++j)
            y[i * 18 + 2 + j] = (uint8_t)((q[j] & 0x0f) | ((q[j + 16] & 0x0f) << 4));
    }
}

void or_dequantize_row_q8_0(const void* vx, float* y, int64_t k) {
    const unsigned char* x = (const unsigned char*)vx;
    for (int64_t i = 0; i < k / QK; ++i) {
        uint16_t dh; memcpy(&dh, x + i * 34, 2);
        const float d = or_fp16_to_fp32(dh);
        for (int j = 0; j < QK; ++j) y[i * QK + j] = (float)(int8_t)x[i * 34 + 2 + j] * d;
    }
}

void or_dequantize_row_q4_0(const void* vx, float* y, int64_t k) {
    const unsigned char* x = (const unsigned char*)vx;
    for (int64_t i = 0; i < k / QK; ++i) {
        uint16_t dh; memcpy(&dh, x + i * 18, 2);
        const float d = or_fp16_to_fp32(dh);
        for (int j = 0; j < QK / 2; ++j) {
            const int x0 = (x[i * 18 + 2 + j] & 0x0f) - 8;
            const int x1 = (x[i * 18 + 2 + j] >> 4) - 8;
            y[i * QK + j] = (float)x0 * d;
            y[i * QK + j + QK / 2] = (float)x1 * d;
        }
    }
}

/* ---------------------------------------------------------------- mul_mat --- */

/* exact integer block dot (vec_dot_q8_0_q8_0 / vec_dot_q4_0_q8_0, ggml-cpu/quants.c:225-256,451-479) */
static double row_dot(int wtype, const unsigned char* w, const unsigned char* a, int64_t nb) {
    double acc = 0.0;
    for (int64_t b = 0; b < nb; ++b) {
        uint16_t dwh, dah;
        int32_t isum = 0;
        const unsigned char* ab = a + b * 34;
        memcpy(&dah, ab, 2);
        if (wtype == 8) {
            const unsigned char* wb = w + b * 34;
            memcpy(&dwh, wb, 2);
            for (int j = 0; j < QK; ++j) isum += (int32_t)(int8_t)wb[2 + j] * (int32_t)(int8_t)ab[2 + j];
        } else {
            const unsigned char* wb = w + b * 18;
            memcpy(&dwh, wb, 2);
            for (int j = 0; j < QK / 2; ++j) {
                const int v0 = (wb[2 + j] & 0x0f) - 8;
                const int v1 = (wb[2 + j] >> 4) - 8;
                isum += v0 * (int32_t)(int8_t)ab[2 + j] + v1 * (int32_t)(int8_t)ab[2 + j + QK / 2];
            }
        }
        acc += (double)(or_fp16_to_fp32(dwh) * or_fp16_to_fp32(dah)) * (double)isum;
    }
    return acc;
}

typedef struct {
    int wtype; const unsigned char* w; const unsigned char* xq; int64_t K, N, M, n0, n1; float* y;
} mm_job;

static void* mm_worker(void* p) {
    mm_job* j = (mm_job*)p;
    const int64_t nb = j->K / QK;
    const int64_t wrow = nb * (j->wtype == 8 ? 34 : 18);
    for (int64_t m = 0; m < j->M; ++m)
        for (int64_t n = j->n0; n < j->n1; ++n)
            j->y[m * j->N + n] = (float)row_dot(j->wtype, j->w + n * wrow, j->xq + m * nb * 34, nb);
    return NULL;
}

int or_mul_mat_q8act(int wtype, const void* w, int64_t K, int64_t N, const void* xq, int64_t M,
                     float* y, int n_threads) {
    if ((wtype != 8 && wtype != 2) || K % QK) return -1;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    pthread_t th[64];
    mm_job jobs[64];
    const int64_t per = (N + n_threads - 1) / n_threads;
    int started = 0;
    for (int t = 0; t < n_threads; ++t) {
        jobs[t] = (mm_job){wtype, (const unsigned char*)w, (const unsigned char*)xq, K, N, M,
                           t * per, (t + 1) * per < N ? (t + 1) * per : N, y};
        if (jobs[t].n0 >= jobs[t].n1) break;
        if (n_threads == 1) { mm_worker(&jobs[t]); continue; }
        pthread_create(&th[t], NULL, mm_worker, &jobs[t]);
        started++;
    }
    for (int t = 0; t < started; ++t) pthread_join(th[t], NULL);
    return 0;
}

int or_mul_mat(int wtype, const void* w, int64_t K, int64_t N, const float* x, int64_t M,
               float* y, int n_threads) {
    if (K % QK) return -1;
    unsigned char* xq = (unsigned char*)malloc((size_t)M * (K / QK) * 34);
    if (!xq) return -1;
    for (int64_t m = 0; m < M; ++m) or_quantize_row_q8_0(x + m * K, xq + m * (K / QK) * 34, K);
    const int r = or_mul_mat_q8act(wtype, w, K, N, xq, M, y, n_threads);
    free(xq);
    return r;
}

/* --------------------------------------------------------------- set_rows --- */

int or_set_rows_f32_f16(uint16_t* dst, int64_t hd, int64_t max_ctx, int64_t H, int64_t B,
                        const float* src, int64_t s, const int64_t* idx) {
    for (int64_t i = 0; i < s; ++i)
        if (idx[i] < 0 || idx[i] >= max_ctx) return -1;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t h = 0; h < H; ++h)
            for (int64_t i = 0; i < s; ++i) {
                const float* sr = src + ((b * H + h) * s + i) * hd;
                uint16_t* dr = dst + ((b * H + h) * max_ctx + idx[i]) * hd;
                for (int64_t c = 0; c < hd; ++c) dr[c] = or_fp32_to_fp16(sr[c]);
            }
    return 0;
}

/* ------------------------------------------------------------- attention --- */

/* One q row over kv range [c0, c1) with the reference's one_chunk arithmetic
 * (ops.cpp:8532-8768): Q in fp16, K.Q accumulated in float, fp16 V accumulator.
 * Leaves M, S and the fp32 copy of the accumulator in *Mo, *So, vkq. */
static void fa_row_ref(const float* qrow, int64_t hd, const uint16_t* kbase, const uint16_t* vbase,
                       const uint16_t* mrow, int64_t c0, int64_t c1, float scale, float* Mo,
                       float* So, float* vkq, uint16_t* q16, uint16_t* acc16) {
    for (int64_t d = 0; d < hd; ++d) { q16[d] = or_fp32_to_fp16(qrow[d]); acc16[d] = 0; }
    float S = 0.0f, M = -INFINITY;
    for (int64_t ic = c0; ic < c1; ++ic) {
        const float mv = mrow ? or_fp16_to_fp32(mrow[ic]) : 0.0f;
        if (mv == -INFINITY) continue;
        const uint16_t* kr = kbase + ic * hd;
        double dot = 0.0;
        for (int64_t d = 0; d < hd; ++d) dot += (double)or_fp16_to_fp32(kr[d]) * or_fp16_to_fp32(q16[d]);
        float sv = (float)dot;
        sv = sv * scale;
        sv += mv;
        const float Mold = M;
        float ms = 1.0f, vs = 1.0f;
        if (sv > M) {
            M = sv;
            ms = expf(Mold - M);
            for (int64_t d = 0; d < hd; ++d) acc16[d] = or_fp32_to_fp16(or_fp16_to_fp32(acc16[d]) * ms);
        } else {
            vs = expf(sv - M);
        }
        const uint16_t* vr = vbase + ic * hd;
        for (int64_t d = 0; d < hd; ++d)
            acc16[d] = or_fp32_to_fp16(fmaf(or_fp16_to_fp32(vr[d]), vs, or_fp16_to_fp32(acc16[d])));
        S = S * ms + vs;
    }
    for (int64_t d = 0; d < hd; ++d) vkq[d] = or_fp16_to_fp32(acc16[d]);
    *Mo = M;
    *So = S;
}

int or_flash_attn_ext_f16(const float* q, int64_t hd, int64_t s, int64_t Hq,
                          const uint16_t* kc, const uint16_t* vc, int64_t max_ctx, int64_t Hkv,
                          int64_t n_kv, const uint16_t* mask, float scale, float* out, int mode,
                          int n_split) {
    if (Hq % Hkv || n_kv > max_ctx || n_kv < 1) return -1;
    const int64_t grp = Hq / Hkv;
    float* vkq = (float*)malloc(sizeof(float) * hd * 2);
    uint16_t* q16 = (uint16_t*)malloc(sizeof(uint16_t) * hd * 2);
    double* accd = (double*)malloc(sizeof(double) * hd);
    double* sc = (double*)malloc(sizeof(double) * n_kv);
    if (!vkq || !q16 || !accd || !sc) return -1;
    uint16_t* acc16 = q16 + hd;
    float* fin = vkq + hd;
    for (int64_t i = 0; i < s; ++i) {
        const uint16_t* mrow = mask ? mask + i * n_kv : NULL;
        for (int64_t h = 0; h < Hq; ++h) {
            const float* qrow = q + (h * s + i) * hd;
            const uint16_t* kb = kc + (h / grp) * max_ctx * hd;
            const uint16_t* vb = vc + (h / grp) * max_ctx * hd;
            float* orow = out + (i * Hq + h) * hd;
            if (mode == 1) {
                double mx = -INFINITY;
                for (int64_t c = 0; c < n_kv; ++c) {
                    double dot = 0.0;
                    for (int64_t d = 0; d < hd; ++d) dot += (double)qrow[d] * or_fp16_to_fp32(kb[c * hd + d]);
                    sc[c] = dot * scale + (mrow ? or_fp16_to_fp32(mrow[c]) : 0.0);
                    if (sc[c] > mx) mx = sc[c];
                }
                double sum = 0.0;
                for (int64_t d = 0; d < hd; ++d) accd[d] = 0.0;
                for (int64_t c = 0; c < n_kv; ++c) {
                    if (sc[c] == -INFINITY) continue;
                    const double p = exp(sc[c] - mx);
                    sum += p;
                    for (int64_t d = 0; d < hd; ++d) accd[d] += p * or_fp16_to_fp32(vb[c * hd + d]);
                }
                for (int64_t d = 0; d < hd; ++d) orow[d] = sum > 0 ? (float)(accd[d] / sum) : 0.0f;
                continue;
            }
            if (s >= 64) {
                /* tiled fp32 path (ops.cpp:8770-9058): fp32 Q, fp32 accumulation — the
                 * exact softmax is its mathematical target; evaluate in double. */
                double mx = -INFINITY;
                for (int64_t c = 0; c < n_kv; ++c) {
                    double dot = 0.0;
                    for (int64_t d = 0; d < hd; ++d) dot += (double)qrow[d] * or_fp16_to_fp32(kb[c * hd + d]);
                    sc[c] = (double)((float)dot * scale) + (mrow ? or_fp16_to_fp32(mrow[c]) : 0.0);
                    if (sc[c] > mx) mx = sc[c];
                }
                double sum = 0.0;
                for (int64_t d = 0; d < hd; ++d) accd[d] = 0.0;
                for (int64_t c = 0; c < n_kv; ++c) {
                    const double p = exp(sc[c] - mx);
                    sum += p;
                    for (int64_t d = 0; d < hd; ++d) accd[d] += p * or_fp16_to_fp32(vb[c * hd + d]);
                }
                for (int64_t d = 0; d < hd; ++d) orow[d] = sum > 0 ? (float)(accd[d] / sum) : 0.0f;
                continue;
            }
            const int split = (s == 1 && n_kv >= 512 && n_split > 1);
            if (!split) {
                float M, S;
                fa_row_ref(qrow, hd, kb, vb, mrow, 0, n_kv, scale, &M, &S, vkq, q16, acc16);
                const float sinv = S == 0.0f ? 0.0f : 1.0f / S;
                for (int64_t d = 0; d < hd; ++d) orow[d] = vkq[d] * sinv;
            } else {
                /* split-KV decode (ops.cpp:9179-9209) + partial reduce (:9060-9128) */
                const int64_t cs = (n_kv + n_split - 1) / n_split;
                float Mf = -INFINITY, Sf = 0.0f;
                for (int64_t d = 0; d < hd; ++d) fin[d] = 0.0f;
                for (int64_t c0 = 0; c0 < n_kv; c0 += cs) {
                    const int64_t c1 = c0 + cs < n_kv ? c0 + cs : n_kv;
                    float Mc, Sc;
                    fa_row_ref(qrow, hd, kb, vb, mrow, c0, c1, scale, &Mc, &Sc, vkq, q16, acc16);
                    if (Sc == 0.0f) continue;
                    const float Mn = fmaxf(Mf, Mc);
                    const float so = expf(Mf - Mn), sn = expf(Mc - Mn);
                    for (int64_t d = 0; d < hd; ++d) fin[d] = fin[d] * so + vkq[d] * sn;
                    Sf = Sf * so + Sc * sn;
                    Mf = Mn;
                }
                const float sinv = Sf != 0.0f ? 1.0f / Sf : 1.0f;
                for (int64_t d = 0; d < hd; ++d) orow[d] = fin[d] * sinv;
            }
        }
    }
    free(vkq); free(q16); free(accd); free(sc);
    return 0;
}

/* -------------------------------------------------------------- soft_max --- */

int or_soft_max_f32(const float* x, int64_t ncols, int64_t nrows, const uint16_t* mask,
                    float scale, float* y) {
    for (int64_t r = 0; r < nrows; ++r) {
        const float* xr = x + r * ncols;
        float* yr = y + r * ncols;
        float mx = -INFINITY;
        for (int64_t c = 0; c < ncols; ++c) {
            float v = xr[c] * scale;
            if (mask) v += or_fp16_to_fp32(mask[r * ncols + c]);
            yr[c] = v;
            if (v > mx) mx = v;
        }
        double sum = 0.0;
        for (int64_t c = 0; c < ncols; ++c) {
            const float e = expf(yr[c] - mx);
            yr[c] = e;
            sum += (double)e;
        }
        const float inv = (float)(1.0 / sum);
        for (int64_t c = 0; c < ncols; ++c) yr[c] *= inv;
    }
    return 0;
}

/* ------------------------------------------------------- executor helpers --- */

int64_t or_pad_kv_len(int64_t n_kv, int64_t max_ctx, int64_t n_pad) {
    if (n_kv < 1) n_kv = 1;
    if (n_pad <= 1) return n_kv < max_ctx ? n_kv : max_ctx;
    int64_t padded = ((n_kv + n_pad - 1) / n_pad) * n_pad;
    if (padded < n_pad) padded = n_pad;
    if (padded > max_ctx) padded = max_ctx;
    return padded;
}

void or_fill_causal_mask_f16(uint16_t* mask, int64_t pos, int64_t s_q, int64_t s_kv) {
    const uint16_t zero = or_fp32_to_fp16(0.0f);
    const uint16_t neg = or_fp32_to_fp16(-32768.0f);
    for (int64_t i = 0; i < s_q; ++i)
        for (int64_t j = 0; j < s_kv; ++j) mask[i * s_kv + j] = (j <= pos + i) ? zero : neg;
}
