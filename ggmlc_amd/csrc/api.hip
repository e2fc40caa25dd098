// extern "C" entry points of libgq.so (declared in include/gq.h): argument
// validation against the ggml op contracts, workspace carving and dispatch to
// the kernels. Validation failures return an error before anything is
// launched, so a rejected call leaves all device state untouched.
#include <atomic>
#include <cmath>
#include <cstdio>

#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace gq {

static thread_local std::string g_err;
static std::atomic<int> g_opt_separate_merge{0};
static std::atomic<int> g_opt_i8_ring{0};

bool option_attn_separate_merge() { return g_opt_separate_merge.load(std::memory_order_relaxed) != 0; }
bool option_gemm_i8_ring() { return g_opt_i8_ring.load(std::memory_order_relaxed) != 0; }

void set_error(const std::string& msg) { g_err = msg; }

int fail(int code, const std::string& msg) {
    set_error(msg);
    return code;
}

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return GQ_OK;
    return fail(GQ_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

namespace {

int64_t block_bytes(int t) { return t == GQ_TYPE_Q8_0 ? Q8_BYTES : (t == GQ_TYPE_Q4_0 ? Q4_BYTES : 0); }

std::string shape(const gq_tensor* t) {
    char buf[160];
    snprintf(buf, sizeof(buf), "type=%d ne=[%lld,%lld,%lld,%lld] nb=[%zu,%zu,%zu,%zu]", t->type,
             (long long)t->ne[0], (long long)t->ne[1], (long long)t->ne[2], (long long)t->ne[3], t->nb[0], t->nb[1],
             t->nb[2], t->nb[3]);
    return buf;
}

// rows of a 4-d tensor addressed as one uniform stride (dims 1..3 collapse)
bool rows_uniform(const gq_tensor* t) {
    return (t->ne[2] == 1 || t->nb[2] == t->nb[1] * (size_t)t->ne[1]) &&
           (t->ne[3] == 1 || t->nb[3] == t->nb[2] * (size_t)t->ne[2]);
}

struct MulMatPlan {
    int64_t K, N, M, x_stride, ldd;
    bool use_gemv;
    bool use_i8;  // 5..16 rows on int8 MFMA (gemm_i8) when the weight is 16-byte aligned
    size_t ws, ws_act;
    size_t ws_rs;  // offset of the GEMM's activation row scales (M floats) in the workspace
};

int plan_mul_mat(const gq_tensor* a, const gq_tensor* b, const gq_tensor* dst, MulMatPlan& p) {
    if (!a || !b) return fail(GQ_ERR_INVALID, "mul_mat: null tensor");
    if (a->type != GQ_TYPE_Q8_0 && a->type != GQ_TYPE_Q4_0)
        return fail(GQ_ERR_UNSUPPORTED, "mul_mat: weight type must be Q8_0 or Q4_0, got " + shape(a));
    if (b->type != GQ_TYPE_F32) return fail(GQ_ERR_UNSUPPORTED, "mul_mat: src1 must be F32, got " + shape(b));
    const int64_t K = a->ne[0], N = a->ne[1];
    if (K <= 0 || K % QK != 0 || N <= 0 || a->ne[2] != 1 || a->ne[3] != 1)
        return fail(GQ_ERR_INVALID, "mul_mat: weight must be [K % 32 == 0, N, 1, 1]: " + shape(a));
    const int64_t bb = block_bytes(a->type);
    if (a->nb[0] != (size_t)bb || a->nb[1] != (size_t)(K / QK * bb))
        return fail(GQ_ERR_INVALID, "mul_mat: weight rows must be contiguous blocks: " + shape(a));
    if (b->ne[0] != K)
        return fail(GQ_ERR_INVALID, "mul_mat shape error: in0 " + shape(a) + " in1 " + shape(b));
    if (b->nb[0] != 4 || b->nb[1] % 4 != 0 || !rows_uniform(b))
        return fail(GQ_ERR_INVALID, "mul_mat: src1 rows must be contiguous and uniformly strided: " + shape(b));
    p.K = K;
    p.N = N;
    p.M = b->ne[1] * b->ne[2] * b->ne[3];
    p.x_stride = (int64_t)(b->nb[1] / 4);
    if (dst) {
        if (dst->type != GQ_TYPE_F32 || dst->ne[0] != N || dst->ne[1] != b->ne[1] || dst->ne[2] != b->ne[2] ||
            dst->ne[3] != b->ne[3])
            return fail(GQ_ERR_INVALID, "mul_mat: dst must be F32 [N, M, ...]: " + shape(dst));
        if (dst->nb[0] != 4 || dst->nb[1] % 4 != 0 || !rows_uniform(dst))
            return fail(GQ_ERR_INVALID, "mul_mat: dst rows must be uniformly strided: " + shape(dst));
        p.ldd = (int64_t)(dst->nb[1] / 4);
    }
    p.use_gemv = p.M <= GEMV_MAX_M;  // GEMV up to this many activation rows, MFMA GEMM above
    // the GEMV quantizes the activation in LDS; the GEMM takes it from the workspace as the
    // exact fp16 pair hi + lo of d * q / r (rows of 2K halves), then the row scales r (M
    // floats), followed by the split-K partials when its plan splits K
    p.use_i8 = !p.use_gemv && p.M <= GEMM_I8_MAX_M && K % GEMM_I8_K_ALIGN == 0 && K <= PREP_MAX_K;
    const size_t raw = p.use_gemv ? 0 : (size_t)p.M * K * 4;
    p.ws_rs = (raw + 255) & ~(size_t)255;
    p.ws_act = p.ws_rs + (p.use_gemv ? 0 : (((size_t)p.M * 4 + 255) & ~(size_t)255));
    p.ws = p.ws_act;
    if (!p.use_gemv && p.M > 0) p.ws += (gemm_plan(N, K, p.M).part_bytes + 255) & ~(size_t)255;
    // the int8 path's activation layout; the GEMM path's size is kept for weights that are
    // not 16-byte aligned (known only at the call), which take the GEMM
    if (p.use_i8) p.ws = std::max(p.ws, (gemm_i8_act_bytes(K) + 255) & ~(size_t)255);
    return GQ_OK;
}

}  // namespace
}  // namespace gq

using namespace gq;

extern "C" {

int gq_abi_version(void) { return GQ_ABI_VERSION; }

const char* gq_last_error(void) { return g_err.c_str(); }

int gq_init(void) {
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    hipDeviceProp_t prop;
    rc = check_hip(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
    if (rc) return rc;
    if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0)
        return fail(GQ_ERR_UNSUPPORTED, std::string("libgq is built for gfx950, device is ") + prop.gcnArchName);
    // the device address of gq_flash_attn_ext_noalloc's static scratch on this device
    return attn_scratch_init(nullptr);
}

int gq_set_option(int option, int64_t value) {
    switch (option) {
        case GQ_OPT_ATTN_SEPARATE_MERGE:
            if (value != 0 && value != 1) return fail(GQ_ERR_INVALID, "set_option: value must be 0 or 1");
            g_opt_separate_merge.store((int)value, std::memory_order_relaxed);
            return GQ_OK;
        case GQ_OPT_GEMM_I8_RING:
            if (value != 0 && value != 1) return fail(GQ_ERR_INVALID, "set_option: value must be 0 or 1");
            g_opt_i8_ring.store((int)value, std::memory_order_relaxed);
            return GQ_OK;
        default:
            return fail(GQ_ERR_INVALID, "set_option: unknown option " + std::to_string(option));
    }
}

int gq_quantize_row_q8_0(const float* x, void* y, int64_t k, gq_stream_t stream) {
    if (k < 0 || k % QK) return fail(GQ_ERR_INVALID, "quantize_row_q8_0: k must be a multiple of 32");
    if (k == 0) return GQ_OK;
    if (!x || !y) return fail(GQ_ERR_INVALID, "quantize_row_q8_0: null pointer");
    if ((reinterpret_cast<uintptr_t>(y) & 1) != 0) return fail(GQ_ERR_INVALID, "quantize_row_q8_0: y must be 2-byte aligned");
    // one row of k elements == k/32 independent blocks
    return quantize_q8_0_blocks(x, 1, k, k, y, (hipStream_t)stream);
}

int gq_quantize_weights(int type, const float* x, void* y, int64_t n, gq_stream_t stream) {
    if (type != GQ_TYPE_Q8_0 && type != GQ_TYPE_Q4_0)
        return fail(GQ_ERR_UNSUPPORTED, "quantize_weights: type must be Q8_0 or Q4_0");
    if (n < 0 || n % QK) return fail(GQ_ERR_INVALID, "quantize_weights: n must be a multiple of 32");
    if (n && (!x || !y)) return fail(GQ_ERR_INVALID, "quantize_weights: null pointer");
    return quantize_weights(type, x, y, n, (hipStream_t)stream);
}

size_t gq_mul_mat_workspace_size(const gq_tensor* a, const gq_tensor* b) {
    MulMatPlan p;
    if (plan_mul_mat(a, b, nullptr, p) != GQ_OK) return 0;
    return p.ws;
}

int gq_mul_mat(const gq_tensor* a, const gq_tensor* b, gq_tensor* dst, void* workspace, size_t workspace_bytes,
               gq_stream_t stream) {
    MulMatPlan p;
    if (!dst) return fail(GQ_ERR_INVALID, "mul_mat: null dst");
    int rc = plan_mul_mat(a, b, dst, p);
    if (rc) return rc;
    if (p.M == 0) return GQ_OK;
    if (p.ws && (!workspace || workspace_bytes < p.ws))
        return fail(GQ_ERR_WORKSPACE, "mul_mat: workspace too small (need " + std::to_string(p.ws) + " bytes)");
    if (p.ws && (reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
        return fail(GQ_ERR_INVALID, "mul_mat: workspace must be 256-byte aligned");
    if ((reinterpret_cast<uintptr_t>(a->data) & 3) != 0)
        return fail(GQ_ERR_INVALID, "mul_mat: weight data must be 4-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    const float* x = static_cast<const float*>(b->data);
    float* y = static_cast<float*>(dst->data);
    const uint8_t* W = static_cast<const uint8_t*>(a->data);
    if (p.use_gemv) return gemv(a->type, W, p.N, p.K, ActSrc{x, p.x_stride, nullptr, 0, nullptr, 0}, p.M, y, p.ldd,
                                GemvFuse{}, s);
    if (p.use_i8 && (reinterpret_cast<uintptr_t>(W) & 15) == 0) {
        uint8_t* act = static_cast<uint8_t*>(workspace);
        rc = act_prep_i8(ActPrep{x, p.x_stride, nullptr, 0, nullptr, 0, p.K, 0, 0, 0.0f}, p.M, act, s);
        if (rc) return rc;
        return gemm_i8(a->type, W, p.N, p.K, act, p.M, y, p.ldd, s);
    }
    uint16_t* A = static_cast<uint16_t*>(workspace);
    float* rs = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + p.ws_rs);
    if (p.K <= PREP_MAX_K)  // one launch: the row in registers, its scale from the quantized blocks
        rc = act_prep(ActPrep{x, p.x_stride, nullptr, 0, nullptr, 0, p.K, 0, 0, 0.0f}, p.M, A, 2 * p.K, rs, s);
    else
        rc = quantize_q8_0_f16(x, p.M, p.K, p.x_stride, A, 2 * p.K, rs, s);
    if (rc) return rc;
    float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + p.ws_act);
    return gemm(a->type, W, p.N, p.K, A, 2 * p.K, rs, p.M, y, p.ldd, part, s);
}

// The rope + KV-store epilogue of gq_mul_mat_fused: the checks of gq_rope_kv_store
// for q/k/v given as the rows of the product, plus the pairing conditions.
static int rope_kv_epilogue(const gq_rope_kv_epilogue& e, const MulMatPlan& p, const gq_tensor* b, GemvFuse& fz) {
    const int64_t hd = e.head_dim, Hq = e.n_head, Hkv = e.n_head_kv, S = p.M;
    if (hd <= 0 || Hq <= 0 || Hkv <= 0 || p.N != (Hq + 2 * Hkv) * hd)
        return fail(GQ_ERR_INVALID, "mul_mat_fused: rope_kv heads do not match the product rows: N = " +
                                        std::to_string(p.N));
    if (b->ne[2] != 1 || b->ne[3] != 1) return fail(GQ_ERR_INVALID, "mul_mat_fused: rope_kv needs b [K, M, 1, 1]");
    if (!e.pos || !e.kv_idx || !e.q_out || !e.k_cache || !e.v_cache)
        return fail(GQ_ERR_INVALID, "mul_mat_fused: rope_kv: null tensor");
    const gq_tensor *qo = e.q_out, *kc = e.k_cache, *vc = e.v_cache;
    if (qo->type != GQ_TYPE_F32 || qo->nb[0] != 4 || qo->ne[0] != hd || qo->ne[1] != Hq || qo->ne[2] != S ||
        qo->ne[3] != 1)
        return fail(GQ_ERR_INVALID, "mul_mat_fused: rope_kv q_out must be F32 [hd, n_head, M, 1]: " + shape(qo));
    for (const gq_tensor* t : {kc, vc})
        if (t->type != GQ_TYPE_F16 || t->nb[0] != 2 || t->ne[0] != hd || t->ne[2] != Hkv || t->ne[3] != 1 ||
            t->ne[1] != kc->ne[1])
            return fail(GQ_ERR_INVALID, "mul_mat_fused: rope_kv caches must be F16 [hd, rows, n_head_kv, 1]: " +
                                            shape(t));
    if (e.pos->type != GQ_TYPE_I32 || e.pos->ne[0] < S || e.pos->nb[0] != 4 || e.kv_idx->type != GQ_TYPE_I64 ||
        e.kv_idx->ne[0] != S || e.kv_idx->nb[0] != 8)
        return fail(GQ_ERR_INVALID, "mul_mat_fused: rope_kv pos must be I32 [>= M], kv_idx I64 [M]");
    if (e.mode != 0 && e.mode != 2) return fail(GQ_ERR_UNSUPPORTED, "mul_mat_fused: rope_kv modes 0 and 2 only");
    if (e.n_dims <= 0 || e.n_dims % 2 || e.n_dims > hd) return fail(GQ_ERR_INVALID, "mul_mat_fused: rope_kv bad n_dims");
    if (hd < 4 || (hd & (hd - 1)) || (e.mode == 2 && e.n_dims != hd))
        return fail(GQ_ERR_UNSUPPORTED,
                    "mul_mat_fused: rope_kv needs a power-of-two head_dim >= 4 and (mode 2) n_dims == head_dim");
    GemvRope& r = fz.rp;
    r.pos = static_cast<const int32_t*>(e.pos->data);
    r.cache = nullptr;
    r.cache_nb1 = 0;
    if (const gq_tensor* c = e.rope_cache) {
        if (c->type != GQ_TYPE_F32 || c->nb[0] != 4 || c->ne[0] != e.n_dims || c->ne[1] < S || c->nb[1] % 8)
            return fail(GQ_ERR_INVALID, "mul_mat_fused: rope_cache must be F32 [n_dims, >= M]: " + shape(c));
        r.cache = static_cast<const float*>(c->data);
        r.cache_nb1 = (int64_t)c->nb[1];
    }
    r.hd = hd, r.Hq = Hq, r.Hkv = Hkv;
    r.hd_log2 = 0;
    while ((int64_t)1 << r.hd_log2 < hd) ++r.hd_log2;
    r.n_dims = e.n_dims, r.neox = e.mode == 2;
    r.theta_scale = powf(e.freq_base, -2.0f / e.n_dims);
    r.freq_scale = e.freq_scale, r.attn_factor = e.attn_factor;
    r.qo = static_cast<float*>(qo->data), r.qonb1 = (int64_t)qo->nb[1], r.qonb2 = (int64_t)qo->nb[2];
    r.kc = static_cast<uint16_t*>(kc->data), r.kcnb1 = (int64_t)kc->nb[1], r.kcnb2 = (int64_t)kc->nb[2];
    r.vc = static_cast<uint16_t*>(vc->data), r.vcnb1 = (int64_t)vc->nb[1], r.vcnb2 = (int64_t)vc->nb[2];
    r.rows = kc->ne[1];
    r.idx = static_cast<const int64_t*>(e.kv_idx->data);
    r.n_bad = e.n_bad;
    fz.rope = 1;
    fz.pair_lo = r.neox ? hd - 1 : 0;
    fz.pair_h = r.neox ? hd / 2 : 0;
    return GQ_OK;
}

// the bias of MUL_MAT's bias ADD: F32 [N] (one row, broadcast over the activation rows)
static int fused_bias(const gq_mul_mat_fusion* f, const MulMatPlan& p, const float** out) {
    *out = nullptr;
    if (!f->bias) return GQ_OK;
    const gq_tensor* t = f->bias;
    if (t->type != GQ_TYPE_F32 || t->ne[0] != p.N || t->ne[1] != 1 || t->ne[2] != 1 || t->ne[3] != 1 ||
        t->nb[0] != 4 || !t->data)
        return fail(GQ_ERR_INVALID, "mul_mat_fused: bias must be F32 [N, 1, 1, 1] with N = " + std::to_string(p.N) +
                                        ": " + shape(t));
    *out = static_cast<const float*>(t->data);
    return GQ_OK;
}

// a pair of slabs [ne0, M, 2, 1] for b's M rows (b 2-d): slab h at data + h * nb[2], rows
// at nb[1] within a slab, the slabs apart; *slab = nb[2] in floats
static int halves_slabs(const gq_tensor* t, int64_t ne0, const gq_tensor* b, const char* what, int64_t* slab) {
    if (!t || t->type != GQ_TYPE_F32 || !t->data || t->ne[0] != ne0 || t->ne[1] != b->ne[1] || t->ne[2] != 2 ||
        t->ne[3] != 1 || b->ne[2] != 1 || b->ne[3] != 1 || t->nb[0] != 4 || t->nb[1] % 4 != 0 ||
        t->nb[2] % 4 != 0 || t->nb[2] < t->nb[1] * (size_t)t->ne[1] || t->nb[1] < (size_t)ne0 * 4)
        return fail(GQ_ERR_INVALID, std::string("mul_mat_fused: ") + what + " halves must be F32 [" +
                                        std::to_string(ne0) + ", M, 2, 1] of disjoint slabs (b 2-d): " +
                                        (t ? shape(t) : std::string("NULL")));
    *slab = (int64_t)(t->nb[2] / 4);
    return GQ_OK;
}

// b as the product's input: with b_swiglu its rows hold 2K values and the input is
// SWIGLU of their halves, so the plan sees the first half; int8 takes the int8 path for
// 1..16 rows (also 1..4, where the GEMV is the default)
static int fused_plan(const gq_tensor* a, const gq_tensor* b, const gq_mul_mat_fusion* f, MulMatPlan& p) {
    if (!f || !a || !b) return fail(GQ_ERR_INVALID, "mul_mat_fused: null argument");
    int rc;
    if (!f->b_swiglu) {
        rc = plan_mul_mat(a, b, nullptr, p);
    } else {
        if (b->ne[0] != 2 * a->ne[0])
            return fail(GQ_ERR_INVALID, "mul_mat_fused: b_swiglu needs b rows of 2K values: " + shape(b));
        gq_tensor h = *b;
        h.ne[0] = a->ne[0];
        rc = plan_mul_mat(a, &h, nullptr, p);
    }
    if (rc || !f->int8) return rc;
    if (p.M > GEMM_I8_MAX_M || p.K % GEMM_I8_K_ALIGN || p.K > PREP_MAX_K ||
        (reinterpret_cast<uintptr_t>(a->data) & 15) != 0)
        return fail(GQ_ERR_UNSUPPORTED, "mul_mat_fused: int8 needs at most 16 rows, K % 256 == 0 (K <= 16384) and "
                                        "16-byte aligned weights");
    p.use_gemv = false;
    p.use_i8 = true;
    p.ws = (gemm_i8_act_bytes(p.K) + 255) & ~(size_t)255;
    return GQ_OK;
}

size_t gq_q8_rows_bytes(int64_t K) { return K > 0 && K % QK == 0 ? gemm_i8_act_bytes(K) : 0; }

int gq_mul_mat_fused_halves(const gq_tensor* a, const gq_tensor* b, const gq_mul_mat_fusion* f) {
    MulMatPlan p;
    if (int rc = fused_plan(a, b, f, p)) return rc;
    if (p.use_gemv || !p.use_i8 || (reinterpret_cast<uintptr_t>(a->data) & 15) != 0 || f->swiglu || f->rope_kv ||
        f->add)
        return 0;
    return !f->bias && gemm_i8_halves(p.N, p.K) ? 1 : 0;
}

size_t gq_mul_mat_fused_workspace_size(const gq_tensor* a, const gq_tensor* b, const gq_mul_mat_fusion* f) {
    MulMatPlan p;
    if (fused_plan(a, b, f, p) != GQ_OK || p.use_gemv) return 0;
    return p.ws;
}

// the GEMM path (M > 4): the input-side fusions run in the activation prologue that
// feeds the GEMM (act_prep); on the int8 path SWIGLU (with the next product's quantized
// rows) and ROPE + SET_ROWS also run as the product's epilogue, and b may come already
// quantized (b_q8)
static int mul_mat_fused_gemm(const gq_tensor* a, const gq_tensor* b, gq_tensor* dst, const gq_mul_mat_fusion* f,
                              const MulMatPlan& p, hipStream_t s) {
    const bool i8 = p.use_i8 && (reinterpret_cast<uintptr_t>(a->data) & 15) == 0;
    if (f->add)
        return fail(GQ_ERR_UNSUPPORTED, "mul_mat_fused: add needs the GEMV path (M <= 4, no int8), M = " +
                                            std::to_string(p.M));
    if ((f->swiglu || f->rope_kv) && !i8)
        return fail(GQ_ERR_UNSUPPORTED, "mul_mat_fused: swiglu / rope_kv need M <= 4 or the int8 path (M <= 16, "
                                        "K % 256 == 0, 16-byte aligned weights), M = " + std::to_string(p.M));
    if (f->out_q8 && !(i8 && f->swiglu))
        return fail(GQ_ERR_INVALID, "mul_mat_fused: out_q8 needs swiglu on the int8 path");
    if (f->b_q8 && !i8) return fail(GQ_ERR_INVALID, "mul_mat_fused: b_q8 needs the int8 path");
    if (f->b_q8 && (f->rms_norm || f->b_add || f->b_swiglu || f->b_sum))
        return fail(GQ_ERR_INVALID, "mul_mat_fused: b_q8 excludes the input-side fusions");
    if (p.K > PREP_MAX_K) return fail(GQ_ERR_UNSUPPORTED, "mul_mat_fused: K above the prologue's limit");
    if (f->b_swiglu && (f->rms_norm || f->b_add))
        return fail(GQ_ERR_INVALID, "mul_mat_fused: b_swiglu excludes rms_norm and b_add");
    const float* bias = nullptr;
    if (int rc = fused_bias(f, p, &bias)) return rc;
    I8Epi epi;
    if (f->rope_kv) {
        GemvFuse fz;
        if (int rc = rope_kv_epilogue(*f->rope_kv, p, b, fz)) return rc;
        epi.rope = 1;
        epi.rp = fz.rp;
        epi.pair_lo = fz.pair_lo;
        epi.pair_h = fz.pair_h;
    } else if (f->swiglu) {
        if (p.N % 2) return fail(GQ_ERR_INVALID, "mul_mat_fused: swiglu needs an even row count: " + shape(a));
        epi.glu = 1;
        epi.pair_lo = ~(int64_t)0;
        epi.pair_h = p.N / 2;
        epi.q8 = static_cast<uint8_t*>(f->out_q8);
    }
    const int64_t n_out = f->swiglu ? p.N / 2 : p.N;
    const bool no_dst = f->rope_kv || (f->out_q8 && !dst);
    if (f->out_halves) {
        if (!i8 || f->swiglu || f->rope_kv || bias || !gemm_i8_halves(p.N, p.K))
            return fail(GQ_ERR_INVALID, "mul_mat_fused: out_halves where the int8 path does not take K in halves "
                                        "(gq_mul_mat_fused_halves)");
        if (int rc = halves_slabs(dst, p.N, b, "dst", &epi.slab)) return rc;
    } else if (!no_dst && (!dst || dst->type != GQ_TYPE_F32 || dst->ne[0] != n_out || dst->ne[1] != b->ne[1] ||
                    dst->ne[2] != b->ne[2] || dst->ne[3] != b->ne[3] || dst->nb[0] != 4 || dst->nb[1] % 4 != 0 ||
                    !rows_uniform(dst)))
        return fail(GQ_ERR_INVALID, "mul_mat_fused: dst must be F32 [" + std::to_string(n_out) + ", M, ...]: " +
                                        (dst ? shape(dst) : std::string("NULL")));
    float* dp = dst && !f->rope_kv ? static_cast<float*>(dst->data) : nullptr;
    const int64_t ldd = dp ? (int64_t)(dst->nb[1] / 4) : 0;
    ActPrep ap{static_cast<const float*>(b->data), p.x_stride, nullptr, 0, nullptr, 0, p.K,
               f->rms_norm ? 1 : 0, f->b_swiglu ? 1 : 0, f->rms_eps};
    if (f->b_add) {
        const gq_tensor* r = f->b_add;
        if (f->b_add_halves) {
            int64_t slab = 0;
            if (int rc = halves_slabs(r, p.K, b, "b_add", &slab)) return rc;
            ap.d2 = static_cast<const float*>(r->data) + slab;
        } else if (r->type != GQ_TYPE_F32 || r->ne[0] != p.K || r->ne[1] != b->ne[1] || r->ne[2] != b->ne[2] ||
                   r->ne[3] != b->ne[3] || r->nb[0] != 4 || r->nb[1] % 4 != 0 || !rows_uniform(r)) {
            return fail(GQ_ERR_INVALID, "mul_mat_fused: b_add must be F32 shaped like b: " + shape(r));
        }
        ap.d = static_cast<const float*>(r->data);
        ap.ds = (int64_t)(r->nb[1] / 4);
        if (f->b_sum) {
            const gq_tensor* o = f->b_sum;
            if (o->type != GQ_TYPE_F32 || o->ne[0] != p.K || o->ne[1] != b->ne[1] || o->ne[2] != b->ne[2] ||
                o->ne[3] != b->ne[3] || o->nb[0] != 4 || o->nb[1] % 4 != 0 || !rows_uniform(o))
                return fail(GQ_ERR_INVALID, "mul_mat_fused: b_sum must be F32 shaped like b: " + shape(o));
            if (o->data == b->data || o->data == r->data || (ap.d2 && o->data == ap.d2))
                return fail(GQ_ERR_INVALID, "mul_mat_fused: b_sum must not alias b or b_add");
            ap.sum = static_cast<float*>(o->data);
            ap.ss = (int64_t)(o->nb[1] / 4);
        }
    } else if (f->b_sum || f->b_add_halves) {
        return fail(GQ_ERR_INVALID, "mul_mat_fused: b_sum and b_add_halves need b_add");
    }
    if (p.M == 0) return GQ_OK;
    if (i8) {
        const uint8_t* act = static_cast<const uint8_t*>(f->b_q8);
        if (!act) {
            if (!f->workspace || f->workspace_bytes < p.ws)
                return fail(GQ_ERR_WORKSPACE,
                            "mul_mat_fused: workspace too small (need " + std::to_string(p.ws) + " bytes)");
            if ((reinterpret_cast<uintptr_t>(f->workspace) & 255) != 0)
                return fail(GQ_ERR_INVALID, "mul_mat_fused: workspace must be 256-byte aligned");
            uint8_t* w = static_cast<uint8_t*>(f->workspace);
            if (int rc = act_prep_i8(ap, p.M, w, s)) return rc;
            act = w;
        }
        return gemm_i8(a->type, static_cast<const uint8_t*>(a->data), p.N, p.K, act, p.M, dp, ldd, s, bias,
                       (epi.rope || epi.glu || epi.slab) ? &epi : nullptr);
    }
    if (!f->workspace || f->workspace_bytes < p.ws)
        return fail(GQ_ERR_WORKSPACE, "mul_mat_fused: workspace too small (need " + std::to_string(p.ws) + " bytes)");
    if ((reinterpret_cast<uintptr_t>(f->workspace) & 255) != 0)
        return fail(GQ_ERR_INVALID, "mul_mat_fused: workspace must be 256-byte aligned");
    if ((reinterpret_cast<uintptr_t>(a->data) & 3) != 0)
        return fail(GQ_ERR_INVALID, "mul_mat_fused: weight data must be 4-byte aligned");
    uint16_t* A = static_cast<uint16_t*>(f->workspace);
    float* rs = reinterpret_cast<float*>(static_cast<uint8_t*>(f->workspace) + p.ws_rs);
    int rc = act_prep(ap, p.M, A, 2 * p.K, rs, s);
    if (rc) return rc;
    float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(f->workspace) + p.ws_act);
    return gemm(a->type, static_cast<const uint8_t*>(a->data), p.N, p.K, A, 2 * p.K, rs, p.M, dp, ldd, part, s,
                bias);
}

int gq_mul_mat_fused(const gq_tensor* a, const gq_tensor* b, gq_tensor* dst, const gq_mul_mat_fusion* f,
                     gq_stream_t stream) {
    if (!f) return fail(GQ_ERR_INVALID, "mul_mat_fused: null fusion");
    if ((f->swiglu != 0) + (f->add != nullptr) + (f->rope_kv != nullptr) > 1)
        return fail(GQ_ERR_INVALID, "mul_mat_fused: swiglu, add and rope_kv are exclusive");
    if (f->rope_kv ? dst != nullptr : (dst == nullptr && !f->out_q8))
        return fail(GQ_ERR_INVALID, "mul_mat_fused: dst must be NULL with rope_kv and given otherwise");
    MulMatPlan p;
    int rc = fused_plan(a, b, f, p);
    if (rc) return rc;
    if (!p.use_gemv) return mul_mat_fused_gemm(a, b, dst, f, p, (hipStream_t)stream);
    if (f->b_swiglu) return fail(GQ_ERR_UNSUPPORTED, "mul_mat_fused: b_swiglu needs M > 4 (use swiglu on the producer)");
    if (f->out_q8 || f->b_q8 || f->out_halves || f->b_add_halves)
        return fail(GQ_ERR_UNSUPPORTED, "mul_mat_fused: out_q8 / b_q8 / out_halves / b_add_halves need M > 4 or "
                                        "int8");
    GemvFuse fz;
    rc = fused_bias(f, p, &fz.bias);
    if (rc) return rc;
    if (f->rope_kv) {
        rc = rope_kv_epilogue(*f->rope_kv, p, b, fz);
        if (rc) return rc;
    } else {
        const int64_t n_out = f->swiglu ? p.N / 2 : p.N;
        if (f->swiglu && p.N % 2)
            return fail(GQ_ERR_INVALID, "mul_mat_fused: swiglu needs an even row count: " + shape(a));
        if (dst->type != GQ_TYPE_F32 || dst->ne[0] != n_out || dst->ne[1] != b->ne[1] || dst->ne[2] != b->ne[2] ||
            dst->ne[3] != b->ne[3] || dst->nb[0] != 4 || dst->nb[1] % 4 != 0 || !rows_uniform(dst))
            return fail(GQ_ERR_INVALID, "mul_mat_fused: dst must be F32 [" + std::to_string(n_out) + ", M, ...]: " +
                                            shape(dst));
    }
    if (f->rms_norm) {
        fz.rms = 1;
        fz.eps = f->rms_eps;
    }
    if (f->swiglu) {
        fz.glu = 1;
        fz.pair_lo = ~(int64_t)0;
        fz.pair_h = p.N / 2;
    }
    if (f->add) {
        const gq_tensor* r = f->add;
        if (r->type != GQ_TYPE_F32 || r->ne[0] != p.N || r->ne[1] != dst->ne[1] || r->ne[2] != dst->ne[2] ||
            r->ne[3] != dst->ne[3] || r->nb[0] != 4 || r->nb[1] % 4 != 0 || !rows_uniform(r))
            return fail(GQ_ERR_INVALID, "mul_mat_fused: add must be F32 shaped like dst: " + shape(r));
        fz.res = static_cast<const float*>(r->data);
        fz.ldr = (int64_t)(r->nb[1] / 4);
    }
    ActSrc act{static_cast<const float*>(b->data), p.x_stride, nullptr, 0, nullptr, 0};
    if (f->b_add) {
        const gq_tensor* r = f->b_add;
        if (r->type != GQ_TYPE_F32 || r->ne[0] != p.K || r->ne[1] != b->ne[1] || r->ne[2] != b->ne[2] ||
            r->ne[3] != b->ne[3] || r->nb[0] != 4 || r->nb[1] % 4 != 0 || !rows_uniform(r))
            return fail(GQ_ERR_INVALID, "mul_mat_fused: b_add must be F32 shaped like b: " + shape(r));
        act.d = static_cast<const float*>(r->data);
        act.ds = (int64_t)(r->nb[1] / 4);
        if (f->b_sum) {
            const gq_tensor* o = f->b_sum;
            if (o->type != GQ_TYPE_F32 || o->ne[0] != p.K || o->ne[1] != b->ne[1] || o->ne[2] != b->ne[2] ||
                o->ne[3] != b->ne[3] || o->nb[0] != 4 || o->nb[1] % 4 != 0 || !rows_uniform(o))
                return fail(GQ_ERR_INVALID, "mul_mat_fused: b_sum must be F32 shaped like b: " + shape(o));
            if (o->data == b->data || o->data == r->data)
                return fail(GQ_ERR_INVALID, "mul_mat_fused: b_sum must not alias b or b_add");
            act.out = static_cast<float*>(o->data);
            act.os = (int64_t)(o->nb[1] / 4);
        }
    } else if (f->b_sum) {
        return fail(GQ_ERR_INVALID, "mul_mat_fused: b_sum needs b_add");
    }
    if (p.M == 0) return GQ_OK;
    if ((reinterpret_cast<uintptr_t>(a->data) & 3) != 0)
        return fail(GQ_ERR_INVALID, "mul_mat_fused: weight data must be 4-byte aligned");
    return gemv(a->type, static_cast<const uint8_t*>(a->data), p.N, p.K, act, p.M,
                dst ? static_cast<float*>(dst->data) : nullptr, dst ? (int64_t)(dst->nb[1] / 4) : 0, fz,
                (hipStream_t)stream);
}

int gq_set_rows(gq_tensor* a, const gq_tensor* b, const gq_tensor* c, int32_t* n_bad, gq_stream_t stream) {
    if (!a || !b || !c) return fail(GQ_ERR_INVALID, "set_rows: null tensor");
    if (a->type != GQ_TYPE_F16 || b->type != GQ_TYPE_F32)
        return fail(GQ_ERR_UNSUPPORTED, "set_rows: supports F32 src into F16 dst: dst " + shape(a) + " src " + shape(b));
    if (c->type != GQ_TYPE_I64 && c->type != GQ_TYPE_I32)
        return fail(GQ_ERR_INVALID, "set_rows: index type must be I64 or I32");
    // ggml.c:3944-3956
    if (a->ne[0] != b->ne[0] || a->ne[2] != b->ne[2] || a->ne[3] != b->ne[3] || b->ne[1] != c->ne[0] ||
        c->ne[1] <= 0 || c->ne[2] <= 0 || b->ne[2] % c->ne[1] != 0 || b->ne[3] % c->ne[2] != 0 || c->ne[3] != 1)
        return fail(GQ_ERR_INVALID, "set_rows: shape mismatch dst " + shape(a) + " src " + shape(b) + " idx " + shape(c));
    if (a->nb[0] != 2 || b->nb[0] != 4) return fail(GQ_ERR_INVALID, "set_rows: rows must be contiguous");
    SetRowsArgs r;
    r.dst = static_cast<uint16_t*>(a->data);
    r.ne0 = a->ne[0];
    r.ne1 = a->ne[1];
    r.ne2 = a->ne[2];
    r.ne3 = a->ne[3];
    r.dnb1 = (int64_t)a->nb[1];
    r.dnb2 = (int64_t)a->nb[2];
    r.dnb3 = (int64_t)a->nb[3];
    r.src = static_cast<const float*>(b->data);
    r.s = b->ne[1];
    r.snb1 = (int64_t)b->nb[1];
    r.snb2 = (int64_t)b->nb[2];
    r.snb3 = (int64_t)b->nb[3];
    r.idx = c->data;
    r.idx64 = c->type == GQ_TYPE_I64;
    r.ine1 = c->ne[1];
    r.ine2 = c->ne[2];
    r.inb0 = (int64_t)c->nb[0];
    r.inb1 = (int64_t)c->nb[1];
    r.inb2 = (int64_t)c->nb[2];
    r.n_bad = n_bad;
    return set_rows_f32_f16(r, (hipStream_t)stream);
}

size_t gq_flash_attn_ext_workspace_size(const gq_tensor* q, const gq_tensor* k) {
    if (!q || !k || k->ne[2] <= 0) return 0;
    return attn_workspace_bytes(q->ne[0], q->ne[1], q->ne[2], k->ne[2], k->ne[1]);
}

}  // extern "C"

namespace {
// validation of a flash_attn_ext call (the op contract of ggml.c:5402-5437) into kernel arguments
int attn_args(const gq_tensor* q, const gq_tensor* k, const gq_tensor* v, const gq_tensor* mask, float scale,
              float max_bias, float logit_softcap, gq_tensor* dst, AttnArgs& a) {
    if (!q || !k || !v || !dst) return fail(GQ_ERR_INVALID, "flash_attn_ext: null tensor");
    if (q->type != GQ_TYPE_F32 || k->type != GQ_TYPE_F16 || v->type != GQ_TYPE_F16 || dst->type != GQ_TYPE_F32)
        return fail(GQ_ERR_UNSUPPORTED, "flash_attn_ext: needs F32 q/dst and F16 k/v");
    const int64_t D = q->ne[0], S = q->ne[1], Hq = q->ne[2], n_kv = k->ne[1], Hkv = k->ne[2];
    if (D < 8 || D > 256 || D % 8)
        return fail(GQ_ERR_UNSUPPORTED, "flash_attn_ext: head dim must be a multiple of 8 up to 256");
    if (k->ne[0] != D || v->ne[0] != D || v->ne[1] != n_kv || v->ne[2] != Hkv || Hkv <= 0 || Hq % Hkv != 0 ||
        q->ne[3] != 1 || k->ne[3] != 1 || v->ne[3] != 1 || n_kv <= 0 || S <= 0)
        return fail(GQ_ERR_INVALID, "flash_attn_ext: shape mismatch q " + shape(q) + " k " + shape(k) + " v " + shape(v));
    if (q->nb[0] != 4 || k->nb[0] != 2 || v->nb[0] != 2 || k->nb[1] % 16 || v->nb[1] % 16 || k->nb[2] % 16 ||
        v->nb[2] % 16 || (reinterpret_cast<uintptr_t>(k->data) & 15) || (reinterpret_cast<uintptr_t>(v->data) & 15))
        return fail(GQ_ERR_INVALID, "flash_attn_ext: k/v rows must be 16-byte aligned");
    if (dst->ne[0] != D || dst->ne[1] != Hq || dst->ne[2] != S || dst->nb[0] != 4 || dst->nb[1] != (size_t)D * 4 ||
        dst->nb[2] != (size_t)D * 4 * Hq)
        return fail(GQ_ERR_INVALID, "flash_attn_ext: dst must be contiguous F32 [D, Hq, S]: " + shape(dst));
    // the kernels address one head's rows through a buffer resource of < 2 GiB
    if ((double)n_kv * (double)k->nb[1] >= 2147418112.0 || (double)n_kv * (double)v->nb[1] >= 2147418112.0)
        return fail(GQ_ERR_INVALID, "flash_attn_ext: one K/V head must span less than 2 GiB: k " + shape(k));
    if (mask) {
        if (mask->type != GQ_TYPE_F16 || mask->ne[0] < n_kv || mask->ne[1] < S || mask->nb[0] != 2 ||
            mask->ne[2] != 1 || mask->ne[3] != 1)
            return fail(GQ_ERR_INVALID, "flash_attn_ext: mask must be F16 [>= n_kv, >= S, 1, 1]: " + shape(mask));
    }
    if (max_bias > 0.0f && !mask) return fail(GQ_ERR_INVALID, "flash_attn_ext: max_bias needs a mask");
    a.q = static_cast<const float*>(q->data);
    a.D = D;
    a.S = S;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.qnb1 = (int64_t)q->nb[1];
    a.qnb2 = (int64_t)q->nb[2];
    a.k = static_cast<const uint16_t*>(k->data);
    a.v = static_cast<const uint16_t*>(v->data);
    a.n_kv = n_kv;
    a.knb1 = (int64_t)k->nb[1];
    a.knb2 = (int64_t)k->nb[2];
    a.vnb1 = (int64_t)v->nb[1];
    a.vnb2 = (int64_t)v->nb[2];
    a.mask = mask ? static_cast<const uint16_t*>(mask->data) : nullptr;
    a.mnb1 = mask ? (int64_t)mask->nb[1] : 0;
    a.scale = scale;
    a.max_bias = max_bias;
    a.softcap = logit_softcap;
    a.dst = static_cast<float*>(dst->data);
    return GQ_OK;
}
}  // namespace

extern "C" {

int gq_flash_attn_ext(const gq_tensor* q, const gq_tensor* k, const gq_tensor* v, const gq_tensor* mask, float scale,
                      float max_bias, float logit_softcap, gq_tensor* dst, void* workspace, size_t workspace_bytes,
                      gq_stream_t stream) {
    AttnArgs a;
    const int rc = attn_args(q, k, v, mask, scale, max_bias, logit_softcap, dst, a);
    if (rc) return rc;
    return attention(a, workspace, workspace_bytes, (hipStream_t)stream);
}

int gq_flash_attn_ext_noalloc(const gq_tensor* q, const gq_tensor* k, const gq_tensor* v, const gq_tensor* mask,
                              float scale, float max_bias, float logit_softcap, gq_tensor* dst, gq_stream_t stream) {
    AttnArgs a;
    const int rc = attn_args(q, k, v, mask, scale, max_bias, logit_softcap, dst, a);
    if (rc) return rc;
    return attention_noalloc(a, (hipStream_t)stream);
}

int gq_attn_reset_counters(gq_stream_t stream) { return attn_reset_counters((hipStream_t)stream); }

int gq_soft_max(const gq_tensor* a, const gq_tensor* mask, float scale, float max_bias, gq_tensor* dst,
                gq_stream_t stream) {
    if (!a || !dst) return fail(GQ_ERR_INVALID, "soft_max: null tensor");
    if (a->type != GQ_TYPE_F32 || dst->type != GQ_TYPE_F32 || a->nb[0] != 4 || dst->nb[0] != 4)
        return fail(GQ_ERR_UNSUPPORTED, "soft_max: needs F32 with contiguous rows");
    for (int i = 0; i < 4; ++i)
        if (a->ne[i] != dst->ne[i]) return fail(GQ_ERR_INVALID, "soft_max: dst shape differs from src");
    SoftmaxArgs s;
    s.x = static_cast<const float*>(a->data);
    s.y = static_cast<float*>(dst->data);
    s.ncols = a->ne[0];
    s.nrows = a->ne[1];
    s.n2 = a->ne[2];
    s.n3 = a->ne[3];
    s.xnb1 = (int64_t)a->nb[1];
    s.xnb2 = (int64_t)a->nb[2];
    s.xnb3 = (int64_t)a->nb[3];
    s.ynb1 = (int64_t)dst->nb[1];
    s.ynb2 = (int64_t)dst->nb[2];
    s.ynb3 = (int64_t)dst->nb[3];
    s.mask = nullptr;
    s.mask_f16 = 0;
    s.mne2 = s.mne3 = 1;
    s.mnb1 = s.mnb2 = s.mnb3 = 0;
    if (mask) {
        if ((mask->type != GQ_TYPE_F16 && mask->type != GQ_TYPE_F32) || mask->ne[0] != a->ne[0] ||
            mask->ne[1] < a->ne[1] || a->ne[2] % mask->ne[2] || a->ne[3] % mask->ne[3])
            return fail(GQ_ERR_INVALID, "soft_max: mask shape " + shape(mask) + " vs " + shape(a));
        s.mask = mask->data;
        s.mask_f16 = mask->type == GQ_TYPE_F16;
        s.mne2 = mask->ne[2];
        s.mne3 = mask->ne[3];
        s.mnb1 = (int64_t)mask->nb[1];
        s.mnb2 = (int64_t)mask->nb[2];
        s.mnb3 = (int64_t)mask->nb[3];
    }
    if (max_bias > 0.0f && !mask) return fail(GQ_ERR_INVALID, "soft_max: max_bias needs a mask");
    s.scale = scale;
    s.max_bias = max_bias;
    return soft_max(s, (hipStream_t)stream);
}

// ---- decoder ops ----------------------------------------------------------

int gq_swiglu(const gq_tensor* a, const gq_tensor* b, gq_tensor* dst, int swapped, gq_stream_t stream) {
    if (!a || !dst) return fail(GQ_ERR_INVALID, "swiglu: null tensor");
    if (a->type != GQ_TYPE_F32 || dst->type != GQ_TYPE_F32 || (b && b->type != GQ_TYPE_F32))
        return fail(GQ_ERR_UNSUPPORTED, "swiglu: F32 only");
    if (a->nb[0] != 4 || dst->nb[0] != 4 || !rows_uniform(a) || !rows_uniform(dst) || (b && (b->nb[0] != 4 || !rows_uniform(b))))
        return fail(GQ_ERR_INVALID, "swiglu: rows must be contiguous and uniformly strided");
    const int64_t nc = b ? a->ne[0] : a->ne[0] / 2;
    const int64_t nrows = a->ne[1] * a->ne[2] * a->ne[3];
    if ((!b && a->ne[0] % 2) || dst->ne[0] != nc || dst->ne[1] * dst->ne[2] * dst->ne[3] != nrows ||
        (b && (b->ne[0] != nc || b->ne[1] * b->ne[2] * b->ne[3] != nrows)))
        return fail(GQ_ERR_INVALID, "swiglu: shape mismatch a " + shape(a) + " dst " + shape(dst));
    const float* A = static_cast<const float*>(a->data);
    const float* x = A;
    const float* g = b ? static_cast<const float*>(b->data) : A + nc;
    int64_t gnb1 = b ? (int64_t)b->nb[1] : (int64_t)a->nb[1];
    if (!b && swapped) {
        x = A + nc;
        g = A;
    }
    return swiglu(x, (int64_t)a->nb[1], g, gnb1, static_cast<float*>(dst->data), (int64_t)dst->nb[1], nc, nrows,
                  (hipStream_t)stream);
}

int gq_rms_norm(const gq_tensor* a, float eps, gq_tensor* dst, gq_stream_t stream) {
    if (!a || !dst) return fail(GQ_ERR_INVALID, "rms_norm: null tensor");
    if (a->type != GQ_TYPE_F32 || dst->type != GQ_TYPE_F32) return fail(GQ_ERR_UNSUPPORTED, "rms_norm: F32 only");
    if (a->nb[0] != 4 || dst->nb[0] != 4 || !rows_uniform(a) || !rows_uniform(dst))
        return fail(GQ_ERR_INVALID, "rms_norm: rows must be contiguous and uniformly strided");
    for (int i = 0; i < 4; ++i)
        if (a->ne[i] != dst->ne[i]) return fail(GQ_ERR_INVALID, "rms_norm: dst shape differs");
    return rms_norm(static_cast<const float*>(a->data), (int64_t)a->nb[1], static_cast<float*>(dst->data),
                    (int64_t)dst->nb[1], a->ne[0], a->ne[1] * a->ne[2] * a->ne[3], eps, (hipStream_t)stream);
}

int gq_rope_ext(const gq_tensor* a, const gq_tensor* pos, int n_dims, int mode, int n_ctx_orig, float freq_base,
                float freq_scale, float ext_factor, float attn_factor, float beta_fast, float beta_slow,
                gq_tensor* dst, gq_stream_t stream) {
    (void)n_ctx_orig;
    (void)beta_fast;
    (void)beta_slow;
    if (!a || !pos || !dst) return fail(GQ_ERR_INVALID, "rope: null tensor");
    if (a->type != GQ_TYPE_F32 || dst->type != GQ_TYPE_F32 || pos->type != GQ_TYPE_I32)
        return fail(GQ_ERR_UNSUPPORTED, "rope: F32 data and I32 positions only");
    if (mode != 0 && mode != 2) return fail(GQ_ERR_UNSUPPORTED, "rope: modes 0 (normal) and 2 (neox) only");
    if (ext_factor != 0.0f) return fail(GQ_ERR_UNSUPPORTED, "rope: YaRN (ext_factor != 0) not implemented");
    if (n_dims <= 0 || n_dims % 2 || n_dims > a->ne[0] || pos->ne[0] < a->ne[2] || a->nb[0] != 4 || dst->nb[0] != 4)
        return fail(GQ_ERR_INVALID, "rope: bad n_dims / positions / strides for " + shape(a));
    for (int i = 0; i < 4; ++i)
        if (a->ne[i] != dst->ne[i]) return fail(GQ_ERR_INVALID, "rope: dst shape differs");
    return rope(static_cast<const float*>(a->data), a->ne[0], a->ne[1], a->ne[2], a->ne[3], (int64_t)a->nb[1],
                (int64_t)a->nb[2], (int64_t)a->nb[3], static_cast<const int32_t*>(pos->data),
                static_cast<float*>(dst->data), (int64_t)dst->nb[1], (int64_t)dst->nb[2], (int64_t)dst->nb[3], n_dims,
                mode == 2, freq_base, freq_scale, attn_factor, (hipStream_t)stream);
}

int gq_rope_kv_store(const gq_tensor* q, const gq_tensor* k, const gq_tensor* v, const gq_tensor* pos, int n_dims,
                     int mode, float freq_base, float freq_scale, float attn_factor, const gq_tensor* kv_idx,
                     gq_tensor* q_out, gq_tensor* k_cache, gq_tensor* v_cache, int32_t* n_bad, gq_stream_t stream) {
    if (!q || !k || !v || !pos || !kv_idx || !q_out || !k_cache || !v_cache)
        return fail(GQ_ERR_INVALID, "rope_kv_store: null tensor");
    for (const gq_tensor* t : {q, k, v, (const gq_tensor*)q_out})
        if (t->type != GQ_TYPE_F32 || t->nb[0] != 4 || t->ne[3] != 1)
            return fail(GQ_ERR_INVALID, "rope_kv_store: q/k/v/q_out must be F32 [hd, H, s, 1] with contiguous rows: " +
                                            shape(t));
    for (const gq_tensor* t : {(const gq_tensor*)k_cache, (const gq_tensor*)v_cache})
        if (t->type != GQ_TYPE_F16 || t->nb[0] != 2 || t->ne[3] != 1)
            return fail(GQ_ERR_INVALID, "rope_kv_store: caches must be F16 [hd, rows, Hkv, 1]: " + shape(t));
    const int64_t hd = q->ne[0], Hq = q->ne[1], Hkv = k->ne[1], S = q->ne[2];
    if (k->ne[0] != hd || v->ne[0] != hd || v->ne[1] != Hkv || k->ne[2] != S || v->ne[2] != S ||
        q_out->ne[0] != hd || q_out->ne[1] != Hq || q_out->ne[2] != S || k_cache->ne[0] != hd ||
        v_cache->ne[0] != hd || k_cache->ne[2] != Hkv || v_cache->ne[2] != Hkv || k_cache->ne[1] != v_cache->ne[1])
        return fail(GQ_ERR_INVALID, "rope_kv_store: shape mismatch q " + shape(q) + " k " + shape(k) + " cache " +
                                        shape(k_cache));
    if (pos->type != GQ_TYPE_I32 || pos->ne[0] < S || pos->nb[0] != 4 || kv_idx->type != GQ_TYPE_I64 ||
        kv_idx->ne[0] != S || kv_idx->nb[0] != 8)
        return fail(GQ_ERR_INVALID, "rope_kv_store: pos must be I32 [>= s], kv_idx I64 [s]");
    if (mode != 0 && mode != 2) return fail(GQ_ERR_UNSUPPORTED, "rope_kv_store: modes 0 (normal) and 2 (neox) only");
    if (n_dims <= 0 || n_dims % 2 || n_dims > hd) return fail(GQ_ERR_INVALID, "rope_kv_store: bad n_dims");
    if ((Hq + Hkv) * hd > 0x7fffffffLL) return fail(GQ_ERR_UNSUPPORTED, "rope_kv_store: (Hq + Hkv) * hd past int32");
    RopeKvArgs a{};
    a.q = static_cast<const float*>(q->data), a.qnb1 = (int64_t)q->nb[1], a.qnb2 = (int64_t)q->nb[2];
    a.k = static_cast<const float*>(k->data), a.knb1 = (int64_t)k->nb[1], a.knb2 = (int64_t)k->nb[2];
    a.v = static_cast<const float*>(v->data), a.vnb1 = (int64_t)v->nb[1], a.vnb2 = (int64_t)v->nb[2];
    a.hd = hd, a.Hq = Hq, a.Hkv = Hkv, a.s = S;
    a.pos = static_cast<const int32_t*>(pos->data);
    a.qo = static_cast<float*>(q_out->data), a.qonb1 = (int64_t)q_out->nb[1], a.qonb2 = (int64_t)q_out->nb[2];
    a.kc = static_cast<uint16_t*>(k_cache->data), a.kcnb1 = (int64_t)k_cache->nb[1], a.kcnb2 = (int64_t)k_cache->nb[2];
    a.vc = static_cast<uint16_t*>(v_cache->data), a.vcnb1 = (int64_t)v_cache->nb[1], a.vcnb2 = (int64_t)v_cache->nb[2];
    a.rows = k_cache->ne[1];
    a.idx = static_cast<const int64_t*>(kv_idx->data);
    a.n_bad = n_bad;
    a.n_dims = n_dims, a.neox = mode == 2;
    a.freq_scale = freq_scale, a.attn_factor = attn_factor;
    return rope_kv(a, freq_base, (hipStream_t)stream);
}

int gq_rope_cache(const gq_tensor* pos, int n_dims, float freq_base, float freq_scale, float attn_factor,
                  gq_tensor* dst, gq_stream_t stream) {
    if (!pos || !dst) return fail(GQ_ERR_INVALID, "rope_cache: null tensor");
    if (pos->type != GQ_TYPE_I32 || pos->nb[0] != 4 || pos->ne[1] != 1 || pos->ne[2] != 1 || pos->ne[3] != 1)
        return fail(GQ_ERR_INVALID, "rope_cache: pos must be I32 [n]");
    if (n_dims <= 0 || n_dims % 2) return fail(GQ_ERR_INVALID, "rope_cache: bad n_dims");
    if (dst->type != GQ_TYPE_F32 || dst->nb[0] != 4 || dst->ne[0] != n_dims || dst->ne[1] != pos->ne[0] ||
        dst->ne[2] != 1 || dst->ne[3] != 1 || dst->nb[1] % 8)
        return fail(GQ_ERR_INVALID, "rope_cache: dst must be F32 [n_dims, n]: " + shape(dst));
    return rope_cache(static_cast<const int32_t*>(pos->data), pos->ne[0], n_dims, freq_base, freq_scale, attn_factor,
                      static_cast<float*>(dst->data), (int64_t)dst->nb[1], (hipStream_t)stream);
}

int gq_add(const gq_tensor* a, const gq_tensor* b, gq_tensor* dst, gq_stream_t stream) {
    if (!a || !b || !dst) return fail(GQ_ERR_INVALID, "add: null tensor");
    if (a->type != GQ_TYPE_F32 || b->type != GQ_TYPE_F32 || dst->type != GQ_TYPE_F32)
        return fail(GQ_ERR_UNSUPPORTED, "add: F32 only");
    for (int i = 0; i < 4; ++i) {
        if (b->ne[i] <= 0 || a->ne[i] % b->ne[i] != 0 || dst->ne[i] != a->ne[i])
            return fail(GQ_ERR_INVALID, "add: b must repeat into a: a " + shape(a) + " b " + shape(b));
    }
    if (a->nb[0] != 4 || b->nb[0] != 4 || dst->nb[0] != 4) return fail(GQ_ERR_INVALID, "add: rows must be contiguous");
    int64_t ane[4], anb[4], bne[4], bnb[4], ynb[4];
    for (int i = 0; i < 4; ++i) {
        ane[i] = a->ne[i];
        anb[i] = (int64_t)a->nb[i];
        bne[i] = b->ne[i];
        bnb[i] = (int64_t)b->nb[i];
        ynb[i] = (int64_t)dst->nb[i];
    }
    return add(static_cast<const float*>(a->data), ane, anb, static_cast<const float*>(b->data), bne, bnb,
               static_cast<float*>(dst->data), ynb, (hipStream_t)stream);
}

int gq_get_rows(const gq_tensor* a, const gq_tensor* b, gq_tensor* dst, gq_stream_t stream) {
    if (!a || !b || !dst) return fail(GQ_ERR_INVALID, "get_rows: null tensor");
    if (a->type != GQ_TYPE_F32 && a->type != GQ_TYPE_F16 && a->type != GQ_TYPE_Q8_0 && a->type != GQ_TYPE_Q4_0)
        return fail(GQ_ERR_UNSUPPORTED, "get_rows: table type must be F32, F16, Q8_0 or Q4_0");
    if (b->type != GQ_TYPE_I32 && b->type != GQ_TYPE_I64) return fail(GQ_ERR_INVALID, "get_rows: ids must be I32/I64");
    if (dst->type != GQ_TYPE_F32 || dst->ne[0] != a->ne[0] || dst->ne[1] != b->ne[0] || a->ne[2] != 1 || a->ne[3] != 1 ||
        b->ne[1] != 1 || b->ne[2] != 1 || dst->nb[0] != 4)
        return fail(GQ_ERR_INVALID, "get_rows: shape mismatch a " + shape(a) + " b " + shape(b) + " dst " + shape(dst));
    if ((a->type == GQ_TYPE_Q8_0 || a->type == GQ_TYPE_Q4_0) && a->ne[0] % QK)
        return fail(GQ_ERR_INVALID, "get_rows: quantized rows must be whole blocks");
    if (b->nb[0] != (size_t)(b->type == GQ_TYPE_I64 ? 8 : 4)) return fail(GQ_ERR_INVALID, "get_rows: ids must be contiguous");
    return get_rows(static_cast<const uint8_t*>(a->data), a->type, a->ne[0], (int64_t)a->nb[1], a->ne[1], b->data,
                    b->type == GQ_TYPE_I64, b->ne[0], static_cast<float*>(dst->data), (int64_t)dst->nb[1],
                    (hipStream_t)stream);
}

int gq_argmax(const gq_tensor* a, gq_tensor* dst, gq_stream_t stream) {
    if (!a || !dst) return fail(GQ_ERR_INVALID, "argmax: null tensor");
    if (a->type != GQ_TYPE_F32 || dst->type != GQ_TYPE_I32 || a->nb[0] != 4 || a->ne[2] != 1 || a->ne[3] != 1 ||
        dst->ne[0] != a->ne[1])
        return fail(GQ_ERR_INVALID, "argmax: a F32 [n, rows] -> dst I32 [rows]");
    return argmax(static_cast<const float*>(a->data), (int64_t)a->nb[1], a->ne[0], a->ne[1],
                  static_cast<int32_t*>(dst->data), (hipStream_t)stream);
}

// ---- persistent-KV step inputs ------------------------------------------------

int gq_kv_step_inputs(const int32_t* pos, int64_t s, int32_t* pos_ids, int64_t* kv_idx, gq_tensor* mask,
                      gq_stream_t stream) {
    if (!pos || s <= 0) return fail(GQ_ERR_INVALID, "kv_step_inputs: needs a device position and s > 0");
    uint16_t* m = nullptr;
    int64_t n_kv = 0, ms = 0;
    if (mask) {
        if (mask->type != GQ_TYPE_F16 || mask->nb[0] != 2 || mask->ne[1] < s || mask->nb[1] % 2)
            return fail(GQ_ERR_INVALID, "kv_step_inputs: mask must be F16 [n_kv, >= s]: " + shape(mask));
        m = static_cast<uint16_t*>(mask->data);
        n_kv = mask->ne[0];
        ms = (int64_t)(mask->nb[1] / 2);
    }
    return kv_step_inputs(pos, s, pos_ids, kv_idx, m, n_kv, ms, (hipStream_t)stream);
}

int gq_kv_advance(int32_t* pos, int64_t s, gq_stream_t stream) {
    if (!pos) return fail(GQ_ERR_INVALID, "kv_advance: null position");
    return kv_advance(pos, s, (hipStream_t)stream);
}

// ---- paged KV (batched decode) ---------------------------------------------

namespace {
int page_log2(int64_t page_size) {
    if (page_size < 64 || (page_size & (page_size - 1)) || page_size > (1 << 20)) return -1;
    int l = 0;
    while ((int64_t(1) << l) < page_size) ++l;
    return l;
}
}  // namespace

size_t gq_flash_attn_paged_workspace_size(const gq_tensor* q, const gq_tensor* k_pool, int64_t max_len,
                                          int64_t page_size) {
    if (!q || !k_pool || k_pool->ne[2] <= 0 || page_log2(page_size) < 0) return 0;
    return attn_paged_workspace_bytes(q->ne[0], q->ne[1], q->ne[2], k_pool->ne[2], max_len, page_size);
}

static int flash_attn_paged_impl(const gq_tensor* q, const gq_tensor* k_pool, const gq_tensor* v_pool,
                                 const gq_tensor* page_table, const gq_tensor* seq_len, int64_t page_size,
                                 int64_t max_len, float scale, gq_tensor* dst, uint8_t* out_q8, void* workspace,
                                 size_t workspace_bytes, gq_stream_t stream) {
    if (!q || !k_pool || !v_pool || !page_table || !seq_len || !dst)
        return fail(GQ_ERR_INVALID, "flash_attn_paged: null tensor");
    if (q->type != GQ_TYPE_F32 || k_pool->type != GQ_TYPE_F16 || v_pool->type != GQ_TYPE_F16 ||
        dst->type != GQ_TYPE_F32 || page_table->type != GQ_TYPE_I32 || seq_len->type != GQ_TYPE_I32)
        return fail(GQ_ERR_UNSUPPORTED, "flash_attn_paged: needs F32 q/dst, F16 pools, I32 page table and lengths");
    const int64_t D = q->ne[0], B = q->ne[1], Hq = q->ne[2], rows = k_pool->ne[1], Hkv = k_pool->ne[2];
    const int lp = page_log2(page_size);
    if (lp < 0) return fail(GQ_ERR_INVALID, "flash_attn_paged: page_size must be a power of two >= 64");
    if (D != 64 && D != 128) return fail(GQ_ERR_UNSUPPORTED, "flash_attn_paged: head dim must be 64 or 128");
    // up to 8 q heads per kv head on any page size, up to 16 with pages of a multiple of 128 rows
    // (the matrix-core kernel)
    if (Hkv <= 0 || Hq % Hkv != 0 || Hq / Hkv > (page_size % 128 == 0 ? 16 : 8))
        return fail(GQ_ERR_UNSUPPORTED, "flash_attn_paged: needs Hq a multiple of Hkv with at most 8 q heads per kv head "
                                        "(16 with pages of a multiple of 128 rows)");
    if (k_pool->ne[0] != D || v_pool->ne[0] != D || v_pool->ne[1] != rows || v_pool->ne[2] != Hkv ||
        q->ne[3] != 1 || k_pool->ne[3] != 1 || v_pool->ne[3] != 1 || B <= 0 || rows <= 0 || max_len <= 0)
        return fail(GQ_ERR_INVALID, "flash_attn_paged: shape mismatch q " + shape(q) + " k " + shape(k_pool) + " v " +
                                        shape(v_pool));
    if (q->nb[0] != 4 || k_pool->nb[0] != 2 || v_pool->nb[0] != 2 || k_pool->nb[1] % 16 || v_pool->nb[1] % 16 ||
        k_pool->nb[2] % 16 || v_pool->nb[2] % 16 || (reinterpret_cast<uintptr_t>(k_pool->data) & 15) ||
        (reinterpret_cast<uintptr_t>(v_pool->data) & 15))
        return fail(GQ_ERR_INVALID, "flash_attn_paged: pool rows must be 16-byte aligned");
    if ((int64_t)k_pool->nb[1] * rows > 0x7fffffff || (int64_t)v_pool->nb[1] * rows > 0x7fffffff)
        return fail(GQ_ERR_INVALID, "flash_attn_paged: one head of a pool must stay below 2 GiB");
    if (page_table->ne[1] < B || page_table->nb[0] != 4 || page_table->nb[1] % 4 || page_table->ne[0] <= 0 ||
        page_table->nb[1] / 4 < (size_t)page_table->ne[0])
        return fail(GQ_ERR_INVALID, "flash_attn_paged: page table must be I32 [max_pages, >= B]: " + shape(page_table));
    if (page_table->ne[0] * page_size < max_len)
        return fail(GQ_ERR_INVALID, "flash_attn_paged: max_len exceeds the page table");
    if (seq_len->ne[0] < B || seq_len->nb[0] != 4)
        return fail(GQ_ERR_INVALID, "flash_attn_paged: seq_len must be I32 [>= B]: " + shape(seq_len));
    if (dst->ne[0] != D || dst->ne[1] != Hq || dst->ne[2] != B || dst->nb[0] != 4 || dst->nb[1] != (size_t)D * 4 ||
        dst->nb[2] != (size_t)D * 4 * Hq)
        return fail(GQ_ERR_INVALID, "flash_attn_paged: dst must be contiguous F32 [D, Hq, B]: " + shape(dst));
    AttnArgs a{};
    a.q = static_cast<const float*>(q->data);
    a.D = D;
    a.S = 1;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.qnb1 = (int64_t)q->nb[1];
    a.qnb2 = (int64_t)q->nb[2];
    a.k = static_cast<const uint16_t*>(k_pool->data);
    a.v = static_cast<const uint16_t*>(v_pool->data);
    a.n_kv = rows;
    a.knb1 = (int64_t)k_pool->nb[1];
    a.knb2 = (int64_t)k_pool->nb[2];
    a.vnb1 = (int64_t)v_pool->nb[1];
    a.vnb2 = (int64_t)v_pool->nb[2];
    a.mask = nullptr;
    a.mnb1 = 0;
    a.scale = scale;
    a.max_bias = 0.0f;
    a.softcap = 0.0f;
    a.dst = static_cast<float*>(dst->data);
    PagedKv pg{static_cast<const int32_t*>(seq_len->data), static_cast<const int32_t*>(page_table->data),
               (int64_t)(page_table->nb[1] / 4), lp, (int)B};
    if (out_q8) {
        if (!attention_paged_q8_ok(D, B, Hq, Hkv, max_len, page_size))
            return fail(GQ_ERR_UNSUPPORTED, "flash_attn_paged_q8: needs B <= 16, 2..16 q heads per kv head on pages "
                                            "of a multiple of 128 rows and max_len > 128");
        if ((reinterpret_cast<uintptr_t>(out_q8) & 15) != 0)
            return fail(GQ_ERR_INVALID, "flash_attn_paged_q8: out_q8 must be 16-byte aligned");
    }
    return attention_paged(a, pg, max_len, workspace, workspace_bytes, (hipStream_t)stream, out_q8);
}

int gq_flash_attn_paged(const gq_tensor* q, const gq_tensor* k_pool, const gq_tensor* v_pool,
                        const gq_tensor* page_table, const gq_tensor* seq_len, int64_t page_size, int64_t max_len,
                        float scale, gq_tensor* dst, void* workspace, size_t workspace_bytes, gq_stream_t stream) {
    return flash_attn_paged_impl(q, k_pool, v_pool, page_table, seq_len, page_size, max_len, scale, dst, nullptr,
                                 workspace, workspace_bytes, stream);
}

int gq_flash_attn_paged_q8(const gq_tensor* q, const gq_tensor* k_pool, const gq_tensor* v_pool,
                           const gq_tensor* page_table, const gq_tensor* seq_len, int64_t page_size, int64_t max_len,
                           float scale, gq_tensor* dst, void* out_q8, void* workspace, size_t workspace_bytes,
                           gq_stream_t stream) {
    if (!out_q8) return fail(GQ_ERR_INVALID, "flash_attn_paged_q8: null out_q8");
    return flash_attn_paged_impl(q, k_pool, v_pool, page_table, seq_len, page_size, max_len, scale, dst,
                                 static_cast<uint8_t*>(out_q8), workspace, workspace_bytes, stream);
}

int gq_paged_step_inputs(const int32_t* pos, int64_t B, const gq_tensor* page_table, int64_t page_size,
                         int64_t trash_row, int64_t* kv_idx, int32_t* seq_len, gq_stream_t stream) {
    const int lp = page_log2(page_size);
    if (!pos || !page_table || !kv_idx || B <= 0 || lp < 0)
        return fail(GQ_ERR_INVALID, "paged_step_inputs: needs positions, a page table, kv_idx and a power-of-two page");
    if (page_table->type != GQ_TYPE_I32 || page_table->ne[1] < B || page_table->nb[0] != 4 || page_table->nb[1] % 4 ||
        page_table->nb[1] / 4 < (size_t)page_table->ne[0])
        return fail(GQ_ERR_INVALID, "paged_step_inputs: page table must be I32 [max_pages, >= B]: " + shape(page_table));
    return paged_step_inputs(pos, B, static_cast<const int32_t*>(page_table->data), (int64_t)(page_table->nb[1] / 4),
                             lp, trash_row, kv_idx, seq_len, (hipStream_t)stream);
}

int gq_paged_advance(int32_t* pos, const int32_t* active, int64_t B, gq_stream_t stream) {
    if (!pos || B < 0) return fail(GQ_ERR_INVALID, "paged_advance: null positions");
    return paged_advance(pos, active, B, (hipStream_t)stream);
}

int gq_kv_pages_copy(gq_tensor* pool, gq_tensor* cache, const int32_t* pages, int64_t n_pages, int64_t page_size,
                     int64_t r0, int64_t r1, int to_pool, gq_stream_t stream) {
    const int lp = page_log2(page_size);
    if (!pool || !cache || !pages || n_pages <= 0 || lp < 0)
        return fail(GQ_ERR_INVALID, "kv_pages_copy: needs a pool, a cache, page ids and a power-of-two page");
    if (pool->type != GQ_TYPE_F16 || cache->type != GQ_TYPE_F16 || pool->ne[0] != cache->ne[0] ||
        pool->ne[2] != cache->ne[2] || pool->ne[3] != 1 || cache->ne[3] != 1 || pool->nb[0] != 2 ||
        cache->nb[0] != 2 || (pool->ne[0] * 2) % 16 || pool->nb[1] % 16 || pool->nb[2] % 16 || cache->nb[1] % 16 ||
        cache->nb[2] % 16 || (reinterpret_cast<uintptr_t>(pool->data) & 15) ||
        (reinterpret_cast<uintptr_t>(cache->data) & 15))
        return fail(GQ_ERR_INVALID, "kv_pages_copy: pool " + shape(pool) + " and cache " + shape(cache) +
                                        " must be F16 [D, rows, H, 1] with 16-byte aligned rows");
    if (r0 < 0 || r1 > cache->ne[1] || r1 > n_pages * page_size)
        return fail(GQ_ERR_INVALID, "kv_pages_copy: row range outside the cache or the pages");
    return kv_pages_copy(static_cast<uint8_t*>(pool->data), (int64_t)pool->nb[1], (int64_t)pool->nb[2], pool->ne[1],
                         static_cast<uint8_t*>(cache->data), (int64_t)cache->nb[1], (int64_t)cache->nb[2], pages,
                         n_pages, lp, r0, r1, pool->ne[2], pool->ne[0] * 2, to_pool, (hipStream_t)stream);
}

}  // extern "C"
