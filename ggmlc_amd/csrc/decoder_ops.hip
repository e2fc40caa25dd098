// The decoder ops around the quantized path (the graph nodes between the
// MUL_MATs and FLASH_ATTN_EXT that ggmlc's executor emits for a LLaMA-style
// layer, runtime/src/executor.cpp:2034-2090, 2355-2357, 2742-2756):
//   GET_ROWS (Q8_0/Q4_0/F16/F32 table -> F32), RMS_NORM, ROPE (normal / NEOX),
//   GLU SWIGLU, ADD (broadcast), ARGMAX.
// Each follows the CPU semantics of ggml-cpu/ops.cpp (cited per kernel); all
// are memory-bound elementwise/row kernels.
#include "common.h"
#include "kernels.h"

namespace gq {

namespace {

__device__ __forceinline__ const uint8_t* at(const void* p, int64_t off) {
    return reinterpret_cast<const uint8_t*>(p) + off;
}

// ---- SWIGLU: y[i] = silu(a[i]) * a[i + nc] per row (ggml_compute_forward_swiglu_f32,
// ops.cpp:3246; swapped exchanges the halves). silu(x) = x / (1 + exp(-x)).
__global__ __launch_bounds__(256) void k_swiglu(const float* __restrict__ a, int64_t anb1, const float* __restrict__ b,
                                                int64_t bnb1, float* __restrict__ y, int64_t ynb1, int64_t nc,
                                                int64_t nrows) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= nc * nrows) return;
    const int64_t r = gid / nc, c = gid % nc;
    const float x = *reinterpret_cast<const float*>(at(a, r * anb1) + c * 4);
    const float g = *reinterpret_cast<const float*>(at(b, r * bnb1) + c * 4);
    *reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(y) + r * ynb1 + c * 4) = swiglu_f(x, g);
}

// ---- RMS_NORM: y = x / sqrt(mean(x^2) + eps) per row (ops.cpp rms_norm_f32, sum in double)
__global__ __launch_bounds__(256) void k_rms_norm(const float* __restrict__ x, int64_t xnb1, float* __restrict__ y,
                                                  int64_t ynb1, int64_t n, float eps) {
    __shared__ double red[4];
    const int64_t r = blockIdx.x;
    const float* xr = reinterpret_cast<const float*>(at(x, r * xnb1));
    float* yr = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(y) + r * ynb1);
    double s = 0.0;
    for (int64_t base = 0; base < n; base += 2048) {  // the order of sumsq8 (shared with the GEMV)
        const int64_t e0 = base + 8 * (int64_t)threadIdx.x;
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = e0 + i < n ? xr[e0 + i] : 0.0f;
        s = sumsq8(v, s);
    }
    const float scale = rms_scale(block_sum_d(s, red), n, eps);
    for (int64_t i = threadIdx.x; i < n; i += 256) yr[i] = xr[i] * scale;
}

// ---- ROPE (ops.cpp:5886-6120, ext_factor = 0): theta_i = p * theta_scale^i built by
// repeated multiplication like ggml_rope_cache_init; NEOX pairs (i, i + n_dims/2),
// NORMAL pairs (2i, 2i+1); dims >= n_dims are copied.
// ---- ROPE cache: (cos, sin) * attn_factor of every rotated pair j < n_dims/2 at each
// position, the table ggml_rope_cache_init fills per position (ops.cpp:5910)
__global__ __launch_bounds__(64) void k_rope_cache(const int32_t* __restrict__ pos, int np, float theta_scale,
                                                   float freq_scale, float attn_factor, float* __restrict__ y,
                                                   int64_t ynb1) {
    const int64_t i = blockIdx.x;
    float* yr = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(y) + i * ynb1);
    const float p = (float)pos[i];
    for (int j = threadIdx.x; j < np; j += blockDim.x) {
        float c, sn;
        rope_cs(p, j, theta_scale, freq_scale, attn_factor, c, sn);
        yr[2 * j] = c;
        yr[2 * j + 1] = sn;
    }
}

__global__ __launch_bounds__(256) void k_rope(const float* __restrict__ x, int64_t ne0, int64_t ne1, int64_t ne2,
                                              int64_t xnb1, int64_t xnb2, int64_t xnb3, const int32_t* __restrict__ pos,
                                              float* __restrict__ y, int64_t ynb1, int64_t ynb2, int64_t ynb3,
                                              int n_dims, int neox, float freq_scale, float attn_factor,
                                              float theta_scale, int64_t total_rows) {
    const int64_t row = blockIdx.x;
    if (row >= total_rows) return;
    const int64_t i1 = row % ne1;
    const int64_t i2 = (row / ne1) % ne2;
    const int64_t i3 = row / (ne1 * ne2);
    const float* xr = reinterpret_cast<const float*>(at(x, i1 * xnb1 + i2 * xnb2 + i3 * xnb3));
    float* yr = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(y) + i1 * ynb1 + i2 * ynb2 + i3 * ynb3);
    const float p = (float)pos[i2];
    const int half = n_dims / 2;
    for (int j = threadIdx.x; j < half; j += blockDim.x) {
        const int i0 = neox ? j : 2 * j;
        const int i1p = neox ? j + half : 2 * j + 1;
        float y0, y1;
        rope_pair(p, j, theta_scale, freq_scale, attn_factor, xr[i0], xr[i1p], y0, y1);
        yr[i0] = y0;
        yr[i1p] = y1;
    }
    for (int64_t j = n_dims + threadIdx.x; j < ne0; j += blockDim.x) yr[j] = xr[j];
}

// ROPE(q), ROPE(k), SET_ROWS(k_cache, k), SET_ROWS(v_cache, v) in one launch: one
// workgroup per token; the token's (cos, sin) pairs are computed once into LDS (the
// rope_cs values every rotating kernel uses) and applied to all its q and k heads, then
// its v heads are copied. Tokens whose cache row is out of range write no k or v and
// count 2 * Hkv (one per head).
__global__ __launch_bounds__(256) void k_rope_kv(RopeKvArgs a) {
    extern __shared__ float2 s_cs[];
    const int64_t i = blockIdx.x;
    const float p = (float)a.pos[i];
    const int half = a.n_dims / 2;
    for (int j = threadIdx.x; j < half; j += blockDim.x) {
        float c, sn;
        rope_cs(p, j, a.theta_scale, a.freq_scale, a.attn_factor, c, sn);
        s_cs[j] = make_float2(c, sn);
    }
    __syncthreads();
    const int64_t row = a.idx[i];
    const bool bad = row < 0 || row >= a.rows;
    if (bad && threadIdx.x == 0 && a.n_bad) atomicAdd(a.n_bad, (int)(2 * a.Hkv));
    // rotated pairs: q heads, then (valid row) k heads. Each thread loads RU pairs before it
    // stores any (the loop otherwise waits for every pair's loads in turn).
    constexpr int RU = 4;
    const int nq = (int)a.Hq * half, nk = bad ? 0 : (int)a.Hkv * half;
    for (int e0 = (int)threadIdx.x; e0 < nq + nk; e0 += (int)blockDim.x * RU) {
        float x0[RU], x1[RU];
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            const int e = e0 + u * (int)blockDim.x;
            x0[u] = x1[u] = 0.0f;
            if (e >= nq + nk) continue;
            const bool isq = e < nq;
            const int ee = isq ? e : e - nq;
            const int h = ee / half, j = ee - h * half;
            const int i0 = a.neox ? j : 2 * j, i1 = a.neox ? j + half : 2 * j + 1;
            const float* xr = isq ? reinterpret_cast<const float*>(at(a.q, i * a.qnb2 + h * a.qnb1))
                                  : reinterpret_cast<const float*>(at(a.k, i * a.knb2 + h * a.knb1));
            x0[u] = xr[i0];
            x1[u] = xr[i1];
        }
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            const int e = e0 + u * (int)blockDim.x;
            if (e >= nq + nk) continue;
            const bool isq = e < nq;
            const int ee = isq ? e : e - nq;
            const int h = ee / half, j = ee - h * half;
            const int i0 = a.neox ? j : 2 * j, i1 = a.neox ? j + half : 2 * j + 1;
            const float2 cs = s_cs[j];
            float y0, y1;
            rope_rotate(cs.x, cs.y, x0[u], x1[u], y0, y1);
            if (isq) {
                float* yr = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(a.qo) + i * a.qonb2 + h * a.qonb1);
                yr[i0] = y0;
                yr[i1] = y1;
            } else {
                uint16_t* yr = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(a.kc) + row * a.kcnb1 + h * a.kcnb2);
                yr[i0] = f2h(y0);
                yr[i1] = f2h(y1);
            }
        }
    }
    // dims past n_dims pass through (q fp32, k fp16)
    const int tail = (int)a.hd - a.n_dims;
    if (tail > 0) {
        for (int e = (int)threadIdx.x; e < (int)(a.Hq + (bad ? 0 : a.Hkv)) * tail; e += (int)blockDim.x) {
            const int h = e / tail, d = a.n_dims + (e - h * tail);
            if (h < a.Hq) {
                const float* xr = reinterpret_cast<const float*>(at(a.q, i * a.qnb2 + h * a.qnb1));
                reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(a.qo) + i * a.qonb2 + h * a.qonb1)[d] = xr[d];
            } else {
                const int kh = h - (int)a.Hq;
                const float* xr = reinterpret_cast<const float*>(at(a.k, i * a.knb2 + kh * a.knb1));
                reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(a.kc) + row * a.kcnb1 + kh * a.kcnb2)[d] =
                    f2h(xr[d]);
            }
        }
    }
    if (bad) return;
    const int hd = (int)a.hd, nv = (int)a.Hkv * hd;
    constexpr int VU = 8;
    for (int e0 = (int)threadIdx.x; e0 < nv; e0 += (int)blockDim.x * VU) {
        float xv[VU];
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int e = e0 + u * (int)blockDim.x;
            xv[u] = 0.0f;
            if (e >= nv) continue;
            const int h = e / hd, d = e - h * hd;
            xv[u] = reinterpret_cast<const float*>(at(a.v, i * a.vnb2 + h * a.vnb1))[d];
        }
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int e = e0 + u * (int)blockDim.x;
            if (e >= nv) continue;
            const int h = e / hd, d = e - h * hd;
            reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(a.vc) + row * a.vcnb1 + h * a.vcnb2)[d] = f2h(xv[u]);
        }
    }
}

// ---- ADD with broadcast of b over a (ggml_can_repeat): y = a + b[i % ne_b]
__global__ __launch_bounds__(256) void k_add(const float* __restrict__ a, const float* __restrict__ b,
                                             float* __restrict__ y, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3,
                                             int64_t anb1, int64_t anb2, int64_t anb3, int64_t bne0, int64_t bne1,
                                             int64_t bne2, int64_t bne3, int64_t bnb1, int64_t bnb2, int64_t bnb3,
                                             int64_t ynb1, int64_t ynb2, int64_t ynb3) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = ne0 * ne1 * ne2 * ne3;
    if (gid >= total) return;
    const int64_t i0 = gid % ne0;
    int64_t r = gid / ne0;
    const int64_t i1 = r % ne1;
    r /= ne1;
    const int64_t i2 = r % ne2;
    const int64_t i3 = r / ne2;
    const float va = *reinterpret_cast<const float*>(at(a, i1 * anb1 + i2 * anb2 + i3 * anb3) + i0 * 4);
    const float vb = *reinterpret_cast<const float*>(
        at(b, (i1 % bne1) * bnb1 + (i2 % bne2) * bnb2 + (i3 % bne3) * bnb3) + (i0 % bne0) * 4);
    *reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(y) + i1 * ynb1 + i2 * ynb2 + i3 * ynb3 + i0 * 4) = va + vb;
}

// ---- GET_ROWS: y[:, i] = dequant(a[:, idx[i]]) (ggml_compute_forward_get_rows_q / _f16 / _f32)
__global__ __launch_bounds__(256) void k_get_rows(const uint8_t* __restrict__ a, int atype, int64_t ne0, int64_t anb1,
                                                  int64_t arows, const void* __restrict__ idx, int idx64,
                                                  int64_t n, float* __restrict__ y, int64_t ynb1) {
    const int64_t i = blockIdx.y;
    if (i >= n) return;
    const int64_t r = idx64 ? reinterpret_cast<const int64_t*>(idx)[i] : reinterpret_cast<const int32_t*>(idx)[i];
    float* yr = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(y) + i * ynb1);
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= ne0) return;
    if (r < 0 || r >= arows) {
        yr[c] = 0.0f;
        return;
    }
    const uint8_t* row = a + r * anb1;
    float v;
    if (atype == GQ_TYPE_F32) {
        v = reinterpret_cast<const float*>(row)[c];
    } else if (atype == GQ_TYPE_F16) {
        v = h2f(reinterpret_cast<const uint16_t*>(row)[c]);
    } else if (atype == GQ_TYPE_Q8_0) {
        const uint8_t* blk = row + (c / QK) * Q8_BYTES;
        v = (float)(int8_t)blk[2 + c % QK] * h2f((uint16_t)(blk[0] | (blk[1] << 8)));
    } else {
        const uint8_t* blk = row + (c / QK) * Q4_BYTES;
        const int j = (int)(c % QK);
        const int qv = j < 16 ? (blk[2 + j] & 0x0f) : (blk[2 + j - 16] >> 4);
        v = (float)(qv - 8) * h2f((uint16_t)(blk[0] | (blk[1] << 8)));
    }
    yr[c] = v;
}

// ---- ARGMAX per row (first index of the maximum, ggml_vec_argmax_f32)
// VEC (16-byte aligned rows, n % 4 == 0): 8 float4 loads in flight per lane per pass
// (32768 values per pass: 5 passes for a 151936-entry vocabulary); otherwise 4 scalar
// loads. Each lane walks its indices in increasing order (the first maximum wins) and
// ties between lanes go to the smaller index.
template <bool VEC>
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, int64_t xnb1, int64_t n,
                                                 int32_t* __restrict__ out) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const int64_t r = blockIdx.x;
    const float* xr = reinterpret_cast<const float*>(at(x, r * xnb1));
    float best = -INFINITY;
    int bi = 0x7fffffff;
    if constexpr (VEC) {
        const float4* x4 = reinterpret_cast<const float4*>(xr);
        const int64_t n4 = n / 4;
        for (int64_t c0 = threadIdx.x; c0 < n4; c0 += 8 * 1024) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t c = c0 + u * 1024;
                v[u] = c < n4 ? x4[c] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = (int)(4 * (c0 + u * 1024));
                if (v[u].x > best) best = v[u].x, bi = i;
                if (v[u].y > best) best = v[u].y, bi = i + 1;
                if (v[u].z > best) best = v[u].z, bi = i + 2;
                if (v[u].w > best) best = v[u].w, bi = i + 3;
            }
        }
    } else {
        for (int64_t i0 = threadIdx.x; i0 < n; i0 += 4 * 1024) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = i0 + u * 1024 < n ? xr[i0 + u * 1024] : -INFINITY;
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (v[u] > best) {
                    best = v[u];
                    bi = (int)(i0 + u * 1024);
                }
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ov > best || (ov == best && oi < bi)) {
            best = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = best;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        best = sv[0];
        bi = si[0];
        for (int w = 1; w < 16; ++w)
            if (sv[w] > best || (sv[w] == best && si[w] < bi)) {
                best = sv[w];
                bi = si[w];
            }
        out[r] = bi == 0x7fffffff ? 0 : bi;
    }
}

}  // namespace

int swiglu(const float* a, int64_t anb1, const float* b, int64_t bnb1, float* y, int64_t ynb1, int64_t nc,
           int64_t nrows, hipStream_t s) {
    const int64_t total = nc * nrows;
    if (total == 0) return GQ_OK;
    hipLaunchKernelGGL(k_swiglu, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, s, a, anb1, b, bnb1, y, ynb1, nc,
                       nrows);
    return check_hip(hipGetLastError(), "swiglu launch");
}

int rms_norm(const float* x, int64_t xnb1, float* y, int64_t ynb1, int64_t n, int64_t nrows, float eps,
             hipStream_t s) {
    if (nrows == 0) return GQ_OK;
    hipLaunchKernelGGL(k_rms_norm, dim3((unsigned)nrows), dim3(256), 0, s, x, xnb1, y, ynb1, n, eps);
    return check_hip(hipGetLastError(), "rms_norm launch");
}

int rope(const float* x, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, int64_t xnb1, int64_t xnb2, int64_t xnb3,
         const int32_t* pos, float* y, int64_t ynb1, int64_t ynb2, int64_t ynb3, int n_dims, int neox, float freq_base,
         float freq_scale, float attn_factor, hipStream_t s) {
    const int64_t rows = ne1 * ne2 * ne3;
    if (rows == 0) return GQ_OK;
    const float theta_scale = powf(freq_base, -2.0f / n_dims);
    hipLaunchKernelGGL(k_rope, dim3((unsigned)rows), dim3(64), 0, s, x, ne0, ne1, ne2, xnb1, xnb2, xnb3, pos, y, ynb1,
                       ynb2, ynb3, n_dims, neox, freq_scale, attn_factor, theta_scale, rows);
    return check_hip(hipGetLastError(), "rope launch");
}

int rope_cache(const int32_t* pos, int64_t n, int n_dims, float freq_base, float freq_scale, float attn_factor,
               float* y, int64_t ynb1, hipStream_t s) {
    if (n == 0) return GQ_OK;
    const float theta_scale = powf(freq_base, -2.0f / n_dims);
    hipLaunchKernelGGL(k_rope_cache, dim3((unsigned)n), dim3(64), 0, s, pos, n_dims / 2, theta_scale, freq_scale,
                       attn_factor, y, ynb1);
    return check_hip(hipGetLastError(), "rope_cache launch");
}

int rope_kv(const RopeKvArgs& a, float freq_base, hipStream_t s) {
    if (a.s == 0) return GQ_OK;
    RopeKvArgs b = a;
    b.theta_scale = powf(freq_base, -2.0f / a.n_dims);
    hipLaunchKernelGGL(k_rope_kv, dim3((unsigned)a.s), dim3(256), (size_t)(a.n_dims / 2) * sizeof(float2), s, b);
    return check_hip(hipGetLastError(), "rope_kv launch");
}

int add(const float* a, const int64_t* ane, const int64_t* anb, const float* b, const int64_t* bne,
        const int64_t* bnb, float* y, const int64_t* ynb, hipStream_t s) {
    const int64_t total = ane[0] * ane[1] * ane[2] * ane[3];
    if (total == 0) return GQ_OK;
    hipLaunchKernelGGL(k_add, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, s, a, b, y, ane[0], ane[1], ane[2],
                       ane[3], anb[1], anb[2], anb[3], bne[0], bne[1], bne[2], bne[3], bnb[1], bnb[2], bnb[3], ynb[1],
                       ynb[2], ynb[3]);
    return check_hip(hipGetLastError(), "add launch");
}

int get_rows(const uint8_t* a, int atype, int64_t ne0, int64_t anb1, int64_t arows, const void* idx, int idx64,
             int64_t n, float* y, int64_t ynb1, hipStream_t s) {
    if (n == 0 || ne0 == 0) return GQ_OK;
    hipLaunchKernelGGL(k_get_rows, dim3((unsigned)cdiv(ne0, 256), (unsigned)n), dim3(256), 0, s, a, atype, ne0, anb1,
                       arows, idx, idx64, n, y, ynb1);
    return check_hip(hipGetLastError(), "get_rows launch");
}

int argmax(const float* x, int64_t xnb1, int64_t n, int64_t nrows, int32_t* out, hipStream_t s) {
    if (nrows == 0) return GQ_OK;
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && xnb1 % 16 == 0 && n % 4 == 0;
    if (vec)
        hipLaunchKernelGGL(k_argmax<true>, dim3((unsigned)nrows), dim3(1024), 0, s, x, xnb1, n, out);
    else
        hipLaunchKernelGGL(k_argmax<false>, dim3((unsigned)nrows), dim3(1024), 0, s, x, xnb1, n, out);
    return check_hip(hipGetLastError(), "argmax launch");
}

}  // namespace gq
