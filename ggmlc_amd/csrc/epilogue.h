// Device-side epilogues shared by the decode GEMV and the int8 MUL_MAT (the output-side
// fusions of gq_mul_mat_fused). Both call the same code, so they give the same bits.
#pragma once

#include "common.h"
#include "kernels.h"

namespace gq {

// Physical weight row of logical row r. Paired epilogues (SWIGLU, rope) need the two rows
// of a pair side by side, so logical rows 2c, 2c+1 of a pair block are the physical rows
// of the pair (pair_lo == 0: the identity).
__device__ __forceinline__ int64_t pair_row(int64_t pair_lo, int64_t pair_h, int64_t r) {
    if (pair_lo == 0) return r;
    return (r & ~pair_lo) + ((r & pair_lo) >> 1) + (r & 1) * pair_h;
}

// Rope epilogue of a fused QKV product for the even logical row `row` of a pair (v0, v1:
// the pair's two dims i0, i1 of head `head`) of activation row m: the work of k_rope_kv
// for those dims with the same arithmetic (q rotated into qo; k rotated, v copied, both
// rounded to fp16 into cache row kv; a bad cache row counted once per token and kv
// head). cs(c) gives the (cos, sin) of rotated pair c at row m's position.
template <typename CsFn>
__device__ __forceinline__ void rope_store(const GemvRope& r, int m, int64_t kv, int64_t row, float v0, float v1,
                                           CsFn cs) {
    const int64_t head = row >> r.hd_log2;
    const int c = (int)((row & (r.hd - 1)) >> 1);
    const int i0 = r.neox ? c : 2 * c;
    const int i1 = r.neox ? c + (int)(r.hd >> 1) : 2 * c + 1;
    float y0 = v0, y1 = v1;
    if (head < r.Hq + r.Hkv && 2 * c < r.n_dims) {
        const float2 t = cs(c);
        rope_rotate(t.x, t.y, v0, v1, y0, y1);
    }
    if (head < r.Hq) {
        float* q = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(r.qo) + m * r.qonb2 + head * r.qonb1);
        q[i0] = y0;
        q[i1] = y1;
        return;
    }
    if (kv < 0 || kv >= r.rows) {
        if (c == 0 && r.n_bad) atomicAdd(r.n_bad, 1);
        return;
    }
    const bool is_k = head < r.Hq + r.Hkv;
    uint16_t* y = is_k ? reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(r.kc) + kv * r.kcnb1 +
                                                      (head - r.Hq) * r.kcnb2)
                       : reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(r.vc) + kv * r.vcnb1 +
                                                      (head - r.Hq - r.Hkv) * r.vcnb2);
    y[i0] = f2h(y0);
    y[i1] = f2h(y1);
}

}  // namespace gq
