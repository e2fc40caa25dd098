// Shared device/host helpers for libgq (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <string>

#include "gq.h"

namespace gq {

// ---- block formats (ggml-common.h:194-199 Q4_0, :251-256 Q8_0) ------------
constexpr int QK = 32;
constexpr int Q8_BYTES = 34;  // fp16 d + 32 x int8
constexpr int Q4_BYTES = 18;  // fp16 d + 16 bytes of nibbles

// Activation layout handed from the quantizer to the GEMV kernels, per token row:
// groups of 8 blocks, each group GS bytes: [256 B int8 qs][8 x (f32 d, i32 sum(qs))][16 B pad].
// The 336-byte stride keeps ds_read_b128 of lanes reading consecutive groups
// free of LDS bank conflicts (84 dwords = 20 mod 32).
constexpr int ACT_GS = 336;
constexpr int ACT_QS_OFF = 0;
constexpr int ACT_DS_OFF = 256;  // (d, s) pairs of the 8 blocks

__host__ __device__ inline int64_t act_row_bytes(int64_t K) { return ((K / QK + 7) / 8) * ACT_GS; }

// ---- error reporting -----------------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_hip(hipError_t e, const char* what);

// ---- device helpers --------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

__device__ __forceinline__ uint16_t f2h(float f) {  // round to nearest even
    _Float16 v = (_Float16)f;
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

// correctly rounded float quotient a/b (double quotient rounded to float is
// innocuous: 53 >= 2*24 + 2)
__device__ __forceinline__ float div_rn(float a, float b) { return (float)((double)a / (double)b); }

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// 16-byte streaming load (nontemporal hint: data is used once)
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

template <int W>
__device__ __forceinline__ float xor_sum(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int W>
__device__ __forceinline__ float xor_max(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// wave-local ordering point for LDS data exchanged between lanes of one wave:
// LDS instructions of a wave execute in order; this keeps the compiler from
// reordering across it.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- lane exchanges without LDS (DPP / permlane) ------------------------------------
// Partner values inside quads of 4 lanes (quad_perm [1,0,3,2] = lane ^ 1 and
// [2,3,0,1] = lane ^ 2), for 32-bit and 64-bit values.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ float quad_xor1(float x) { return __uint_as_float(dpp_u<0xB1>(__float_as_uint(x))); }
__device__ __forceinline__ float quad_xor2(float x) { return __uint_as_float(dpp_u<0x4E>(__float_as_uint(x))); }
__device__ __forceinline__ int quad_xor1(int x) { return (int)dpp_u<0xB1>((uint32_t)x); }
__device__ __forceinline__ int quad_xor2(int x) { return (int)dpp_u<0x4E>((uint32_t)x); }
template <int CTRL>
__device__ __forceinline__ double dpp_d(double x) {
    const uint64_t u = (uint64_t)__builtin_bit_cast(unsigned long long, x);
    const uint64_t r = (uint64_t)dpp_u<CTRL>((uint32_t)u) | ((uint64_t)dpp_u<CTRL>((uint32_t)(u >> 32)) << 32);
    return __builtin_bit_cast(double, (unsigned long long)r);
}
// sum of a double over the 64 lanes of a wave, every lane gets the total: quads
// (lane ^ 1, lane ^ 2), half rows (row_half_mirror), rows of 16 (row_mirror), then
// row pairs and wave halves through permlane16/32 swaps. Each step adds two values
// that every lane of the pair holds, so all lanes end with the same bits.
__device__ __forceinline__ double wave_sum_d(double s) {
    s += dpp_d<0xB1>(s);
    s += dpp_d<0x4E>(s);
    s += dpp_d<0x141>(s);
    s += dpp_d<0x140>(s);
    {
        const uint64_t u = (uint64_t)__builtin_bit_cast(unsigned long long, s);
        const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)u, (uint32_t)u, false, false);
        const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(u >> 32), (uint32_t)(u >> 32), false, false);
        const double a = __builtin_bit_cast(double, (unsigned long long)((uint64_t)lo[0] | ((uint64_t)hi[0] << 32)));
        const double b = __builtin_bit_cast(double, (unsigned long long)((uint64_t)lo[1] | ((uint64_t)hi[1] << 32)));
        s = a + b;
    }
    {
        const uint64_t u = (uint64_t)__builtin_bit_cast(unsigned long long, s);
        const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)u, (uint32_t)u, false, false);
        const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(u >> 32), (uint32_t)(u >> 32), false, false);
        const double a = __builtin_bit_cast(double, (unsigned long long)((uint64_t)lo[0] | ((uint64_t)hi[0] << 32)));
        const double b = __builtin_bit_cast(double, (unsigned long long)((uint64_t)lo[1] | ((uint64_t)hi[1] << 32)));
        s = a + b;
    }
    return s;
}

// ---- RMS_NORM sum of squares in one fixed order ----------------------------------
// Shared by k_rms_norm and the GEMV prologue, so RMS_NORM -> MUL_MAT fused gives the
// bits of the two ops: lane t of a 256-lane block owns elements [2048 p + 8 t,
// 2048 p + 8 t + 8) of pass p; each lane sums the fp32 squares in double in element
// order (passes ascending), then the wave (wave_sum_d), then the 4 waves in order
// (ggml sums in double too: ops.cpp rms_norm_f32, ggml_float).
__device__ __forceinline__ double sumsq8(const float (&v)[8], double s) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float p = v[i] * v[i];
        s += (double)p;
    }
    return s;
}

// all 256 lanes call it; red: 4 doubles of LDS (free again on return)
__device__ __forceinline__ double block_sum_d(double s, double* red) {
    s = wave_sum_d(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const double r = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    return r;
}

// ROPE (ops.cpp:5886-6120, ext_factor = 0) of one pair j at position p: theta =
// p * theta_scale^j built by repeated multiplication like ggml_rope_cache_init,
// then (cos, sin) * attn_factor and the rotation. Every kernel that rotates (k_rope,
// k_rope_kv, the GEMV's rope epilogue) uses these, so all give the same bits.
__device__ __forceinline__ void rope_cs(float p, int j, float theta_scale, float freq_scale, float attn_factor,
                                        float& c, float& s) {
#pragma clang fp contract(off)
    float theta = p;
    for (int t = 0; t < j; ++t) theta *= theta_scale;
    theta *= freq_scale;
    c = cosf(theta) * attn_factor;
    s = sinf(theta) * attn_factor;
}
__device__ __forceinline__ void rope_rotate(float c, float s, float x0, float x1, float& y0, float& y1) {
#pragma clang fp contract(off)
    y0 = x0 * c - x1 * s;
    y1 = x0 * s + x1 * c;
}
__device__ __forceinline__ void rope_pair(float p, int j, float theta_scale, float freq_scale, float attn_factor,
                                          float x0, float x1, float& y0, float& y1) {
    float c, s;
    rope_cs(p, j, theta_scale, freq_scale, attn_factor, c, s);
    rope_rotate(c, s, x0, x1, y0, y1);
}

// SWIGLU of one element: silu(g) * u with ggml's silu(x) = x / (1 + exp(-x))
// (ops.cpp:3246). k_swiglu, the GEMV's SWIGLU epilogue and the GEMM path's prologue
// all use this, so they give the same bits.
__device__ __forceinline__ float swiglu_f(float g, float u) {
    const float sg = g / (1.0f + expf(-g));
    return sg * u;
}

// y = x * rms_scale(...): scale = 1 / sqrt(mean(x^2) + eps), mean rounded to fp32
__device__ __forceinline__ float rms_scale(double sumsq, int64_t n, float eps) {
    const float mean = (float)(sumsq / (double)n);
    return 1.0f / sqrtf(mean + eps);
}

// ---- activation quantizer core ----------------------------------------------
// ggml x86 quantize_row_q8_0 (ggml-cpu/arch/x86/quants.c:302-398) for one 32-wide
// block spread over 4 consecutive lanes of a wave (8 elements each):
//   amax = max|x|, d = fp16_rne(amax / 127), id = amax ? 127 / amax : 0,
//   q = saturate_int8(rne(x * id)).
// Every lane of the wave must call it (xor shuffles); lanes without data pass
// zeros. Returns the lane's 8 quants, the block's fp16 scale bits and the
// block sum of the quants (used by Q4_0 dot products).
// The callers' translation units are built with fp contraction off for this.
__device__ __forceinline__ void quant8_block(const float (&v)[8], int (&q)[8], uint16_t& dh, int& qsum) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, quad_xor1(amax));
    amax = fmaxf(amax, quad_xor2(amax));
    const float d = amax / 127.0f;  // IEEE division, correctly rounded (no fast-math)
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float r = __builtin_rintf(v[i] * id);
        int iv = (int)r;
        iv = iv > 127 ? 127 : (iv < -128 ? -128 : iv);
        q[i] = iv;
        s += iv;
    }
    s += quad_xor1(s);
    s += quad_xor2(s);
    qsum = s;
    dh = f2h(d);
}

// The row scale of the GEMM's fp16 activation pairs: the smallest power of two
// r = 2^e (0 <= e <= 8) with 127 * dmax / r <= 65504, dmax the largest block scale of the
// row (|q| <= 127, so every d * q / r of the row then has a finite fp16 hi part). r = 1
// for every row whose scales stay below 65504 / 127 = 515.8 (amax below ~65500), which
// leaves those rows' pairs as they were. A non-finite dmax (amax / 127 past the fp16
// range: ggml's own scale is then inf) keeps the loop bounded and the products inf.
__device__ __forceinline__ float row_pow2(float dmax) {
    float t = 127.0f * dmax;  // exact: 11 x 7 significant bits
    float r = 1.0f;
#pragma unroll 1
    for (int e = 0; e < 8 && t > 65504.0f; ++e) {
        t *= 0.5f;
        r *= 2.0f;
    }
    return r;
}

// d * q / r of 8 quants of one block as an exact pair of fp16 vectors, hi + lo == d * q / r
// (r = 2^e from row_pow2, inv = 1 / r): d (fp16, 11 significant bits) times |q| <= 127 has
// at most 18 significant bits and is exact in fp32, and so is its power-of-two multiple;
// hi = fp16_rne(d * q / r) (finite: |d * q / r| <= 65504) and lo = d * q / r - hi (exact in
// fp32) has at most 7 significant bits on the grid of (d / r)'s last bit, which fp16 holds
// exactly while that grid is >= 2^-24: always for r = 1 (d normal: the grid is >= 2^-24;
// d subnormal: every product is a multiple of 2^-24), and for r = 2^e > 1 for every block
// with d >= 2^(e - 14), which includes every block within a factor 2^22 of the row's
// largest scale (that one is above 2^(e + 8)). Smaller blocks of such a row round lo to
// the 2^-24 grid, an error below 2^-40 of the row's largest product. Packed two halves
// per dword, element i in the low half of dword i / 2.
__device__ __forceinline__ void split_dq8(const int (&q)[8], uint16_t dh, float inv, uint4& hi, uint4& lo) {
    const float df = h2f(dh) * inv;  // exact: inv is a power of two, d / r stays a normal fp32
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float p0 = (float)q[2 * i] * df, p1 = (float)q[2 * i + 1] * df;
        const uint16_t h0 = f2h(p0), h1 = f2h(p1);
        const uint16_t l0 = f2h(p0 - h2f(h0)), l1 = f2h(p1 - h2f(h1));
        h[i] = h0 | ((uint32_t)h1 << 16);
        l[i] = l0 | ((uint32_t)l1 << 16);
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// load the 8 floats of one lane's part of a block (16-byte loads when aligned)
template <bool VEC>
__device__ __forceinline__ void load8(const float* src, bool valid, float (&v)[8]) {
    if (!valid) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
        return;
    }
    if (VEC) {
        const float4 a0 = *reinterpret_cast<const float4*>(src);
        const float4 a1 = *reinterpret_cast<const float4*>(src + 4);
        v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
        v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = src[i];
    }
}

// The activation rows a GEMV consumes: x, or x + d (an ADD node fused in front; its
// sum is also written to `out` by the workgroup that has `writer` set, since later
// nodes read it).
struct ActSrc {
    const float* x;
    int64_t xs;        // row stride (floats)
    const float* d;    // null: no ADD
    int64_t ds;
    float* out;        // null: the sum is not stored
    int64_t os;
};

template <bool VEC>
__device__ __forceinline__ void act_load8(const ActSrc& a, int m, int64_t e0, bool valid, float (&v)[8]) {
    load8<VEC>(a.x + (int64_t)m * a.xs + e0, valid, v);
    if (a.d) {
        float w[8];
        load8<VEC>(a.d + (int64_t)m * a.ds + e0, valid, w);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = v[i] + w[i];  // ADD(x, d): x + d
    }
}

template <bool VEC>
__device__ __forceinline__ void act_store_sum(const ActSrc& a, bool writer, int m, int64_t e0, bool valid,
                                              const float (&v)[8]) {
    if (!a.out || !writer || !valid) return;
    float* o = a.out + (int64_t)m * a.os + e0;
    if (VEC) {
        *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = v[i];
    }
}

// RMS scales of M activation rows (K % 32 == 0) read from global memory, in the
// order of sumsq8 / block_sum_d; all 256 lanes call it.
template <bool VEC, int MM>
__device__ __forceinline__ void rms_scales(const ActSrc& a, int M, int K, float eps, float (&scale)[MM],
                                           double* red) {
    const int nb = K / QK;
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        if (m >= M) break;
        double s = 0.0;
        for (int base = 0; base < nb * 4; base += 256) {
            const int t = base + (int)threadIdx.x;
            float v[8];
            act_load8<VEC>(a, m, (int64_t)t * 8, (t >> 2) < nb, v);
            s = sumsq8(v, s);
        }
        scale[m] = rms_scale(block_sum_d(s, red), K, eps);
    }
}

// Quantize M activation rows (K elements) into the ACT_GS layout at dst (row stride
// act_bytes), cooperatively by a 256-lane block; row m is multiplied by scale[m]
// first (1 leaves it unchanged: RMS_NORM fusion).
template <bool VEC, int MM = 1>
__device__ __forceinline__ void quantize_rows_to_act(const ActSrc& a, bool writer, int M, int K, uint8_t* dst,
                                                     int act_bytes, const float* scale = nullptr) {
    const int nb = K / QK;
    for (int m = 0; m < M; ++m) {
        const float sc = scale ? scale[m] : 1.0f;
        for (int base = 0; base < nb * 4; base += 256) {
            const int t = base + (int)threadIdx.x;
            const int b = t >> 2, part = t & 3;
            const bool valid = b < nb;
            float v[8];
            act_load8<VEC>(a, m, (int64_t)b * QK + part * 8, valid, v);
            act_store_sum<VEC>(a, writer, m, (int64_t)b * QK + part * 8, valid, v);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = v[i] * sc;
            int q[8];
            uint16_t dh;
            int qsum;
            quant8_block(v, q, dh, qsum);
            if (valid) {
                uint8_t* gp = dst + m * act_bytes + (b >> 3) * ACT_GS;
                const int bi = b & 7;
                uint32_t lo = 0, hi = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    lo |= (uint32_t)(q[i] & 0xff) << (8 * i);
                    hi |= (uint32_t)(q[4 + i] & 0xff) << (8 * i);
                }
                *reinterpret_cast<uint2*>(gp + ACT_QS_OFF + bi * QK + part * 8) = make_uint2(lo, hi);
                if (part == 0) {
                    *reinterpret_cast<float2*>(gp + ACT_DS_OFF + 8 * bi) =
                        make_float2(h2f(dh), __int_as_float(qsum));
                }
            }
        }
    }
}

}  // namespace gq
