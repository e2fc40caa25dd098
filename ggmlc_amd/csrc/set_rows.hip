// SET_ROWS F32 -> F16: the persistent KV-cache write.
//
// Semantics: ggml_compute_forward_set_rows_impl<float, idx_t>
// (ggml-cpu/ops.cpp:5156-5259) with from_float = fp32 -> fp16 round to nearest
// even (ggml_cpu_fp32_to_fp16, ggml-cpu.c:3444-3474):
//   dst[:, idx[i, i2 % ne_c1, i3 % ne_c2], i2, i3] = fp16(src[:, i, i2, i3]).
// One lane converts 4 consecutive elements (16-byte load, 8-byte store) when
// the row length and strides allow it, else 1. Rows whose index is out of range
// are skipped and counted (the reference asserts instead).
#include "common.h"
#include "kernels.h"

namespace gq {

namespace {

template <int VEC>
__global__ __launch_bounds__(256) void k_set_rows(SetRowsArgs a) {
    const int64_t per_row = a.ne0 / VEC;
    const int64_t total = per_row * a.s * a.ne2 * a.ne3;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    const int64_t c = (gid % per_row) * VEC;
    int64_t r = gid / per_row;
    const int64_t i = r % a.s;
    r /= a.s;
    const int64_t i2 = r % a.ne2;
    const int64_t i3 = r / a.ne2;
    const uint8_t* ip = reinterpret_cast<const uint8_t*>(a.idx) + i * a.inb0 + (i2 % a.ine1) * a.inb1 +
                        (i3 % a.ine2) * a.inb2;
    const int64_t row = a.idx64 ? *reinterpret_cast<const int64_t*>(ip) : (int64_t)*reinterpret_cast<const int32_t*>(ip);
    if (row < 0 || row >= a.ne1) {
        if (c == 0 && a.n_bad) atomicAdd(a.n_bad, 1);
        return;
    }
    const float* sp = reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(a.src) + i * a.snb1 +
                                                     i2 * a.snb2 + i3 * a.snb3) + c;
    uint16_t* dp = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(a.dst) + row * a.dnb1 +
                                               i2 * a.dnb2 + i3 * a.dnb3) + c;
    if (VEC == 4) {
        const float4 v = *reinterpret_cast<const float4*>(sp);
        uint2 o;
        o.x = (uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16);
        o.y = (uint32_t)f2h(v.z) | ((uint32_t)f2h(v.w) << 16);
        *reinterpret_cast<uint2*>(dp) = o;
    } else {
        *dp = f2h(*sp);
    }
}

}  // namespace

int set_rows_f32_f16(const SetRowsArgs& a, hipStream_t s) {
    const bool vec = a.ne0 % 4 == 0 && (reinterpret_cast<uintptr_t>(a.src) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(a.dst) & 7) == 0 && a.snb1 % 16 == 0 && a.snb2 % 16 == 0 &&
                     a.snb3 % 16 == 0 && a.dnb1 % 8 == 0 && a.dnb2 % 8 == 0 && a.dnb3 % 8 == 0;
    const int v = vec ? 4 : 1;
    const int64_t total = (a.ne0 / v) * a.s * a.ne2 * a.ne3;
    if (total == 0) return GQ_OK;
    const dim3 grid((unsigned)cdiv(total, 256));
    if (vec)
        hipLaunchKernelGGL(k_set_rows<4>, grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(k_set_rows<1>, grid, dim3(256), 0, s, a);
    return check_hip(hipGetLastError(), "set_rows launch");
}

}  // namespace gq
