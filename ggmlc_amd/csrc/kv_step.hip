// Per-step inputs of the persistent KV path, produced on the device from a
// device-resident position so that a captured decode graph can be replayed
// without host work:
//   pos_ids[i] = kv_idx[i] = pos + i                 (i < s)
//   mask[i][j] = 0 if j <= pos + i else -32768 (fp16) (j < n_kv)
// This is what ggmlc's executor does on the host before each run
// (set_decode_pos / set_chunk_pos, runtime/src/executor.cpp:1181-1393, and
// fill_f16_causal_mask, :136-148, ATTN_MASK_MIN_FP16 = -32768 from
// runtime/include/ggmlc/types.h:240).
//
// The batched paged decode path has its per-slot counterparts: pool rows and
// lengths from per-sequence device positions, the position advance, and the copy of
// a sequence's rows between its pages and a contiguous prefill cache (the role of
// paged_kv_map_existing_pages / the VA-window mapping of executor.cpp:634-886).
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

// Batched paged decode: sequence b writes its token at logical row pos[b], which lives
// at pool row table[b][pos[b] / P] * P + pos[b] % P, and then attends to pos[b] + 1 rows.
__global__ __launch_bounds__(64) void k_paged_step_inputs(const int32_t* __restrict__ pos, int64_t B,
                                                          const int32_t* __restrict__ table, int64_t tstride,
                                                          int log2p, int64_t trash_row, int64_t* __restrict__ kv_idx,
                                                          int32_t* __restrict__ seq_len) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const int64_t p = pos[b];
    const int64_t pi = p >> log2p;
    const int page = (p >= 0 && pi < tstride) ? table[b * tstride + pi] : -1;
    kv_idx[b] = page < 0 ? trash_row : ((int64_t)page << log2p) + (p & ((1 << log2p) - 1));
    if (seq_len) seq_len[b] = page < 0 ? 0 : (int32_t)(p + 1);
}

__global__ __launch_bounds__(64) void k_paged_advance(int32_t* __restrict__ pos, const int32_t* __restrict__ active,
                                                      int64_t B) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B && (active == nullptr || active[b] != 0)) pos[b] += 1;
}

// rows [r0, r1) of a sequence between its contiguous cache (row r) and its pages in a
// pool (row pages[r / P] * P + r % P); 16 bytes per thread, lanes along the row
__global__ __launch_bounds__(256) void k_kv_pages_copy(uint8_t* __restrict__ pool, int64_t pnb1, int64_t pnb2,
                                                       int64_t prows, uint8_t* __restrict__ cache, int64_t cnb1,
                                                       int64_t cnb2, const int32_t* __restrict__ pages,
                                                       int64_t n_pages, int log2p, int64_t r0, int64_t nrows,
                                                       int64_t H, int64_t cpr, int to_pool) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= nrows * H * cpr) return;
    const int64_t c = gid % cpr, t = gid / cpr;
    const int64_t r = r0 + t % nrows, h = t / nrows;
    const int64_t pi = r >> log2p;
    if (pi >= n_pages) return;
    const int page = pages[pi];
    if (page < 0) return;
    const int64_t pr = ((int64_t)page << log2p) + (r & ((1 << log2p) - 1));
    if (pr >= prows) return;
    uint4* pp = reinterpret_cast<uint4*>(pool + h * pnb2 + pr * pnb1) + c;
    uint4* cp = reinterpret_cast<uint4*>(cache + h * cnb2 + r * cnb1) + c;
    if (to_pool) *pp = *cp;
    else *cp = *pp;
}

}  // namespace

int paged_step_inputs(const int32_t* pos, int64_t B, const int32_t* table, int64_t tstride, int log2p,
                      int64_t trash_row, int64_t* kv_idx, int32_t* seq_len, hipStream_t st) {
    if (B == 0) return GQ_OK;
    hipLaunchKernelGGL(k_paged_step_inputs, dim3((unsigned)cdiv(B, 64)), dim3(64), 0, st, pos, B, table, tstride,
                       log2p, trash_row, kv_idx, seq_len);
    return check_hip(hipGetLastError(), "paged_step_inputs launch");
}

int paged_advance(int32_t* pos, const int32_t* active, int64_t B, hipStream_t st) {
    if (B == 0) return GQ_OK;
    hipLaunchKernelGGL(k_paged_advance, dim3((unsigned)cdiv(B, 64)), dim3(64), 0, st, pos, active, B);
    return check_hip(hipGetLastError(), "paged_advance launch");
}

int kv_pages_copy(uint8_t* pool, int64_t pnb1, int64_t pnb2, int64_t prows, uint8_t* cache, int64_t cnb1, int64_t cnb2,
                  const int32_t* pages, int64_t n_pages, int log2p, int64_t r0, int64_t r1, int64_t H,
                  int64_t row_bytes, int to_pool, hipStream_t st) {
    const int64_t nrows = r1 - r0, cpr = row_bytes / 16;
    if (nrows <= 0 || H <= 0) return GQ_OK;
    const int64_t n = nrows * H * cpr;
    hipLaunchKernelGGL(k_kv_pages_copy, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, pool, pnb1, pnb2, prows, cache,
                       cnb1, cnb2, pages, n_pages, log2p, r0, nrows, H, cpr, to_pool);
    return check_hip(hipGetLastError(), "kv_pages_copy launch");
}

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
