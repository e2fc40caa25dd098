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
// groups of 8 blocks, each group GS bytes: [256 B int8 qs][8 x f32 d][8 x i32 sum(qs)][16 B pad].
// The 336-byte stride keeps ds_read_b128 of lanes reading consecutive groups
// free of LDS bank conflicts (84 dwords = 20 mod 32).
constexpr int ACT_GS = 336;
constexpr int ACT_QS_OFF = 0;
constexpr int ACT_D_OFF = 256;
constexpr int ACT_S_OFF = 288;

inline int64_t act_row_bytes(int64_t K) { return ((K / QK + 7) / 8) * ACT_GS; }

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

}  // namespace gq
