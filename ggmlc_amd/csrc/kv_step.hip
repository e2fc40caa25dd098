// Per-step inputs of the persistent KV path, produced on the device from a
// device-resident position so that a captured decode graph can be replayed
// without host work:
//   pos_ids[i] = kv_idx[i] = pos + i                 (i < s)
//   mask[i][j] = 0 if j <= pos + i else -32768 (fp16) (j < n_kv)
// This is what ggmlc's executor does on the host before each run
// (set_decode_pos / set_chunk_pos, runtime/src/executor.cpp:1181-1393, and
// fill_f16_causal_mask, :136-148, ATTN_MASK_MIN_FP16 = -32768 from
// runtime/include/ggmlc/types.h:240).
#include "common.h"
#include "kernels.h"

namespace gq {

namespace {

__global__ __launch_bounds__(256) void k_kv_step_inputs(const int32_t* __restrict__ pos_dev, int64_t s,
                                                        int32_t* __restrict__ pos_ids, int64_t* __restrict__ kv_idx,
                                                        uint16_t* __restrict__ mask, int64_t n_kv,
                                                        int64_t mask_stride) {
    const int64_t pos = pos_dev[0];
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid < s) {
        if (pos_ids) pos_ids[gid] = (int32_t)(pos + gid);
        if (kv_idx) kv_idx[gid] = pos + gid;
    }
    if (mask && gid < s * n_kv) {
        const int64_t i = gid / n_kv, j = gid % n_kv;
        mask[i * mask_stride + j] = (j <= pos + i) ? (uint16_t)0x0000 : (uint16_t)0xF800;  // 0 / -32768
    }
}

__global__ void k_kv_advance(int32_t* pos_dev, int64_t s) { pos_dev[0] += (int32_t)s; }

}  // namespace

int kv_step_inputs(const int32_t* pos_dev, int64_t s, int32_t* pos_ids, int64_t* kv_idx, uint16_t* mask,
                   int64_t n_kv, int64_t mask_stride, hipStream_t st) {
    const int64_t n = s > s * n_kv ? s : (mask ? s * n_kv : s);
    if (n == 0) return GQ_OK;
    hipLaunchKernelGGL(k_kv_step_inputs, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, pos_dev, s, pos_ids, kv_idx,
                       mask, n_kv, mask_stride);
    return check_hip(hipGetLastError(), "kv_step_inputs launch");
}

int kv_advance(int32_t* pos_dev, int64_t s, hipStream_t st) {
    hipLaunchKernelGGL(k_kv_advance, dim3(1), dim3(1), 0, st, pos_dev, s);
    return check_hip(hipGetLastError(), "kv_advance launch");
}

}  // namespace gq
