// Test infrastructure only: a thin C entry layer over the reference's own ggml
// CPU backend (ggml 0.20.2, vendored at third_party/ggml in the reference tree),
// compiled from the reference sources by oracle/Makefile into oracle/_ref/.
//
// Nothing here re-implements an operator: every function builds a one-node ggml
// graph exactly the way ggmlc's executor does (runtime/src/executor.cpp) and runs
// it with ggml_graph_compute_with_ctx on the ggml CPU backend. The product path
// never links or loads this library; only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg do.
//
// Reference call sites mirrored:
//   quantize_row_q8_0  -> ggml_get_type_traits_cpu(Q8_0)->from_float
//                         (ggml-cpu/ggml-cpu.c:271-279, arch/x86/quants.c:302-398)
//   mul_mat            -> ggml_mul_mat (ggml.c:3278), executor.cpp:2362-2447
//   set_rows           -> ggml_set_rows (ggml.c:3937), executor.cpp:2181-2184
//   flash_attn_ext     -> ggml_flash_attn_ext (ggml.c:5402), executor.cpp:2195-2197
//   soft_max           -> ggml_soft_max_ext (ggml.c:4081), executor.cpp:2358-2361
//   whole LLaMA decoder -> the graph the executor builds for a fused LLaMA block
//                         (executor.cpp:1738-2810; KV wiring :2130-2197), run by
//                         ggml_graph_compute on the CPU backend
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "ggml.h"
#include "ggml-alloc.h"
#include "ggml-backend.h"
#include "ggml-cpu.h"

// ggml-quants.h:23 (declared here with an opaque block pointer; same C symbol)
extern "C" void quantize_row_q8_0_ref(const float* x, void* y, int64_t k);

namespace {

struct Ctx {
    ggml_context* ctx = nullptr;
    explicit Ctx(size_t bytes) {
        ggml_init_params p = {bytes + 64 * 1024 * 1024, nullptr, false};
        ctx = ggml_init(p);
    }
    ~Ctx() {
        if (ctx) ggml_free(ctx);
    }
};

int run_graph(ggml_context* ctx, ggml_tensor* out, int n_threads) {
    ggml_cgraph* gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, out);
    return ggml_graph_compute_with_ctx(ctx, gf, n_threads) == GGML_STATUS_SUCCESS ? 0 : -1;
}

}  // namespace

extern "C" {

void ref_init(void) { ggml_cpu_init(); }

const char* ref_ggml_version(void) { return ggml_version(); }

// x86 runtime activation quantizer (the one the CPU backend runs on src1).
void ref_quantize_row_q8_0(const float* x, void* y, int64_t k) {
    ggml_cpu_init();
    ggml_get_type_traits_cpu(GGML_TYPE_Q8_0)->from_float(x, y, k);
}

// ggml's scalar reference quantizers (ggml-quants.c:113-148, 276-299).
void ref_quantize_row_q8_0_ref(const float* x, void* y, int64_t k) {
    quantize_row_q8_0_ref(x, y, k);
}

// dst[M][N] = W(type, N rows of K) x X(M rows of K, fp32). type: 2 = Q4_0, 8 = Q8_0, 1 = F16, 0 = F32.
int ref_mul_mat(int wtype, const void* w, int64_t K, int64_t N, const float* x, int64_t M,
                float* dst, int n_threads) {
    ggml_cpu_init();
    const ggml_type t = (ggml_type)wtype;
    const size_t wbytes = ggml_row_size(t, K) * (size_t)N;
    Ctx c(wbytes + (size_t)(K * M + N * M) * sizeof(float) * 2 + (size_t)K * M);
    if (!c.ctx) return -1;
    ggml_tensor* W = ggml_new_tensor_2d(c.ctx, t, K, N);
    ggml_tensor* X = ggml_new_tensor_2d(c.ctx, GGML_TYPE_F32, K, M);
    memcpy(W->data, w, wbytes);
    memcpy(X->data, x, sizeof(float) * K * M);
    ggml_tensor* Y = ggml_mul_mat(c.ctx, W, X);
    if (run_graph(c.ctx, Y, n_threads) != 0) return -1;
    memcpy(dst, Y->data, sizeof(float) * N * M);
    return 0;
}

// KV-cache row scatter exactly as the executor wires it: dst is the F16 cache
// [hd, max_ctx, H, B] (contiguous), src the F32 rows [hd, s, H, B], idx I64 [s].
// The cache is updated in place (dst is input and output).
int ref_set_rows_f32_f16(uint16_t* cache, int64_t hd, int64_t max_ctx, int64_t H, int64_t B,
                         const float* src, int64_t s, const int64_t* idx, int n_threads) {
    ggml_cpu_init();
    const size_t cache_bytes = sizeof(uint16_t) * hd * max_ctx * H * B;
    Ctx c(cache_bytes + sizeof(float) * hd * s * H * B + sizeof(int64_t) * s);
    if (!c.ctx) return -1;
    ggml_tensor* dst = ggml_new_tensor_4d(c.ctx, GGML_TYPE_F16, hd, max_ctx, H, B);
    ggml_tensor* sr = ggml_new_tensor_4d(c.ctx, GGML_TYPE_F32, hd, s, H, B);
    ggml_tensor* ix = ggml_new_tensor_1d(c.ctx, GGML_TYPE_I64, s);
    memcpy(dst->data, cache, cache_bytes);
    memcpy(sr->data, src, sizeof(float) * hd * s * H * B);
    memcpy(ix->data, idx, sizeof(int64_t) * s);
    ggml_tensor* out = ggml_set_rows(c.ctx, dst, sr, ix);
    if (run_graph(c.ctx, out, n_threads) != 0) return -1;
    memcpy(cache, dst->data, cache_bytes);
    return 0;
}

// FLASH_ATTN_EXT over the active prefix of a padded KV cache, as the executor
// builds it with set_rows (executor.cpp:2143-2197):
//   q    F32 [hd, s, Hq, 1] contiguous
//   kc,vc F16 caches [hd, max_ctx, Hkv, 1]; the op sees views [hd, n_kv, Hkv, 1]
//   mask F16 [n_kv, s] contiguous, or nullptr
//   out  F32 [hd, Hq, s, 1] (permuted layout produced by the op)
int ref_flash_attn_ext_f16(const float* q, int64_t hd, int64_t s, int64_t Hq,
                           const uint16_t* kc, const uint16_t* vc, int64_t max_ctx, int64_t Hkv,
                           int64_t n_kv, const uint16_t* mask, float scale, float* out,
                           int n_threads) {
    ggml_cpu_init();
    const size_t cache_bytes = sizeof(uint16_t) * hd * max_ctx * Hkv;
    Ctx c(2 * cache_bytes + sizeof(float) * hd * s * Hq * 2 + sizeof(uint16_t) * n_kv * s +
          (size_t)16 * 1024 * 1024);
    if (!c.ctx) return -1;
    ggml_tensor* Q = ggml_new_tensor_4d(c.ctx, GGML_TYPE_F32, hd, s, Hq, 1);
    ggml_tensor* KC = ggml_new_tensor_4d(c.ctx, GGML_TYPE_F16, hd, max_ctx, Hkv, 1);
    ggml_tensor* VC = ggml_new_tensor_4d(c.ctx, GGML_TYPE_F16, hd, max_ctx, Hkv, 1);
    memcpy(Q->data, q, sizeof(float) * hd * s * Hq);
    memcpy(KC->data, kc, cache_bytes);
    memcpy(VC->data, vc, cache_bytes);
    ggml_tensor* K = ggml_view_4d(c.ctx, KC, hd, n_kv, Hkv, 1, KC->nb[1], KC->nb[2], KC->nb[3], 0);
    ggml_tensor* V = ggml_view_4d(c.ctx, VC, hd, n_kv, Hkv, 1, VC->nb[1], VC->nb[2], VC->nb[3], 0);
    ggml_tensor* MK = nullptr;
    if (mask) {
        MK = ggml_new_tensor_4d(c.ctx, GGML_TYPE_F16, n_kv, s, 1, 1);
        memcpy(MK->data, mask, sizeof(uint16_t) * n_kv * s);
    }
    ggml_tensor* O = ggml_flash_attn_ext(c.ctx, Q, K, V, MK, scale, 0.0f, 0.0f);
    if (run_graph(c.ctx, O, n_threads) != 0) return -1;
    memcpy(out, O->data, sizeof(float) * hd * Hq * s);
    return 0;
}

// SOFT_MAX: y = softmax(x*scale + mask) per row of ncols; mask F16 [ncols, nrows] or nullptr.
int ref_soft_max_f32(const float* x, int64_t ncols, int64_t nrows, const uint16_t* mask,
                     float scale, float* y, int n_threads) {
    ggml_cpu_init();
    Ctx c(sizeof(float) * ncols * nrows * 2 + sizeof(uint16_t) * ncols * nrows);
    if (!c.ctx) return -1;
    ggml_tensor* X = ggml_new_tensor_2d(c.ctx, GGML_TYPE_F32, ncols, nrows);
    memcpy(X->data, x, sizeof(float) * ncols * nrows);
    ggml_tensor* MK = nullptr;
    if (mask) {
        MK = ggml_new_tensor_2d(c.ctx, GGML_TYPE_F16, ncols, nrows);
        memcpy(MK->data, mask, sizeof(uint16_t) * ncols * nrows);
    }
    ggml_tensor* Y = ggml_soft_max_ext(c.ctx, X, MK, scale, 0.0f);
    if (run_graph(c.ctx, Y, n_threads) != 0) return -1;
    memcpy(y, Y->data, sizeof(float) * ncols * nrows);
    return 0;
}

// ---- persistent graphs for timing the CPU baseline --------------------------
// The weights are copied into the ggml context once; ref_graph_run only copies
// the activation in, runs ggml_graph_compute_with_ctx and copies the result out.

struct RefGraph {
    ggml_context* ctx = nullptr;
    ggml_cgraph* gf = nullptr;
    ggml_tensor* x = nullptr;
    ggml_tensor* y = nullptr;
};

static RefGraph* new_graph(size_t bytes) {
    RefGraph* g = new RefGraph;
    ggml_init_params p = {bytes + 256 * 1024 * 1024, nullptr, false};
    g->ctx = ggml_init(p);
    if (!g->ctx) {
        delete g;
        return nullptr;
    }
    return g;
}

// y[M][N] = W x (the decode GEMV / prefill GEMM node alone)
void* ref_mm_create(int wtype, const void* w, int64_t K, int64_t N, int64_t M) {
    ggml_cpu_init();
    const ggml_type t = (ggml_type)wtype;
    const size_t wbytes = ggml_row_size(t, K) * (size_t)N;
    RefGraph* g = new_graph(wbytes + sizeof(float) * (K + N) * M * 2);
    if (!g) return nullptr;
    ggml_tensor* W = ggml_new_tensor_2d(g->ctx, t, K, N);
    memcpy(W->data, w, wbytes);
    g->x = ggml_new_tensor_2d(g->ctx, GGML_TYPE_F32, K, M);
    g->y = ggml_mul_mat(g->ctx, W, g->x);
    g->gf = ggml_new_graph(g->ctx);
    ggml_build_forward_expand(g->gf, g->y);
    return g;
}

// LLaMA MLP block as ggmlc's fused graph runs it (fusion.py:1224-1546 concatenates
// [W_gate; W_up]): y = W_down . swiglu(W_gate_up . x)   (MUL_MAT -> GLU -> MUL_MAT)
void* ref_mlp_create(int wtype, const void* w_gate_up, const void* w_down, int64_t K, int64_t F, int64_t M) {
    ggml_cpu_init();
    const ggml_type t = (ggml_type)wtype;
    const size_t b1 = ggml_row_size(t, K) * (size_t)(2 * F);
    const size_t b2 = ggml_row_size(t, F) * (size_t)K;
    RefGraph* g = new_graph(b1 + b2 + sizeof(float) * (K + 3 * F + K) * M * 2);
    if (!g) return nullptr;
    ggml_tensor* Wgu = ggml_new_tensor_2d(g->ctx, t, K, 2 * F);
    ggml_tensor* Wd = ggml_new_tensor_2d(g->ctx, t, F, K);
    memcpy(Wgu->data, w_gate_up, b1);
    memcpy(Wd->data, w_down, b2);
    g->x = ggml_new_tensor_2d(g->ctx, GGML_TYPE_F32, K, M);
    ggml_tensor* h = ggml_mul_mat(g->ctx, Wgu, g->x);
    ggml_tensor* a = ggml_swiglu(g->ctx, h);
    g->y = ggml_mul_mat(g->ctx, Wd, a);
    g->gf = ggml_new_graph(g->ctx);
    ggml_build_forward_expand(g->gf, g->y);
    return g;
}

int ref_graph_run(void* h, const float* x, float* y, int n_threads) {
    RefGraph* g = (RefGraph*)h;
    memcpy(g->x->data, x, ggml_nbytes(g->x));
    if (ggml_graph_compute_with_ctx(g->ctx, g->gf, n_threads) != GGML_STATUS_SUCCESS) return -1;
    if (y) memcpy(y, g->y->data, ggml_nbytes(g->y));
    return 0;
}

void ref_graph_free(void* h) {
    RefGraph* g = (RefGraph*)h;
    if (!g) return;
    ggml_free(g->ctx);
    delete g;
}

// ---- decoder ops (one node each, executor.cpp:2034-2090, 2742-2756) -----------

int ref_swiglu(const float* a, int64_t nc, int64_t nrows, float* y) {
    ggml_cpu_init();
    Ctx c(sizeof(float) * nc * nrows * 3);
    ggml_tensor* A = ggml_new_tensor_2d(c.ctx, GGML_TYPE_F32, 2 * nc, nrows);
    memcpy(A->data, a, sizeof(float) * 2 * nc * nrows);
    ggml_tensor* Y = ggml_swiglu(c.ctx, A);
    if (run_graph(c.ctx, Y, 1) != 0) return -1;
    memcpy(y, Y->data, sizeof(float) * nc * nrows);
    return 0;
}

int ref_rms_norm(const float* x, int64_t n, int64_t nrows, float eps, float* y) {
    ggml_cpu_init();
    Ctx c(sizeof(float) * n * nrows * 2);
    ggml_tensor* X = ggml_new_tensor_2d(c.ctx, GGML_TYPE_F32, n, nrows);
    memcpy(X->data, x, sizeof(float) * n * nrows);
    ggml_tensor* Y = ggml_rms_norm(c.ctx, X, eps);
    if (run_graph(c.ctx, Y, 1) != 0) return -1;
    memcpy(y, Y->data, sizeof(float) * n * nrows);
    return 0;
}

// x [hd, heads, seq] F32, pos I32 [seq]
int ref_rope(const float* x, int64_t hd, int64_t heads, int64_t seq, const int32_t* pos, int n_dims, int mode,
             float freq_base, float* y) {
    ggml_cpu_init();
    Ctx c(sizeof(float) * hd * heads * seq * 2 + sizeof(int32_t) * seq);
    ggml_tensor* X = ggml_new_tensor_3d(c.ctx, GGML_TYPE_F32, hd, heads, seq);
    ggml_tensor* P = ggml_new_tensor_1d(c.ctx, GGML_TYPE_I32, seq);
    memcpy(X->data, x, sizeof(float) * hd * heads * seq);
    memcpy(P->data, pos, sizeof(int32_t) * seq);
    ggml_tensor* Y = ggml_rope_ext(c.ctx, X, P, nullptr, n_dims, mode, 0, freq_base, 1.0f, 0.0f, 1.0f, 0.0f, 0.0f);
    if (run_graph(c.ctx, Y, 1) != 0) return -1;
    memcpy(y, Y->data, sizeof(float) * hd * heads * seq);
    return 0;
}

// table [n_embd, rows] of type wtype, ids I32 [n] -> y F32 [n_embd, n]
int ref_get_rows(int wtype, const void* table, int64_t n_embd, int64_t rows, const int32_t* ids, int64_t n, float* y) {
    ggml_cpu_init();
    const ggml_type t = (ggml_type)wtype;
    const size_t tb = ggml_row_size(t, n_embd) * (size_t)rows;
    Ctx c(tb + sizeof(float) * n_embd * n + sizeof(int32_t) * n);
    ggml_tensor* T = ggml_new_tensor_2d(c.ctx, t, n_embd, rows);
    ggml_tensor* I = ggml_new_tensor_1d(c.ctx, GGML_TYPE_I32, n);
    memcpy(T->data, table, tb);
    memcpy(I->data, ids, sizeof(int32_t) * n);
    ggml_tensor* Y = ggml_get_rows(c.ctx, T, I);
    if (run_graph(c.ctx, Y, 1) != 0) return -1;
    memcpy(y, Y->data, sizeof(float) * n_embd * n);
    return 0;
}

int ref_argmax(const float* x, int64_t n, int64_t nrows, int32_t* out) {
    ggml_cpu_init();
    Ctx c(sizeof(float) * n * nrows + sizeof(int32_t) * nrows);
    ggml_tensor* X = ggml_new_tensor_2d(c.ctx, GGML_TYPE_F32, n, nrows);
    memcpy(X->data, x, sizeof(float) * n * nrows);
    ggml_tensor* Y = ggml_argmax(c.ctx, X);
    if (run_graph(c.ctx, Y, 1) != 0) return -1;
    memcpy(out, Y->data, sizeof(int32_t) * nrows);
    return 0;
}

// ---- whole decoder (CPU baseline of the model-level benchmark) -------------------
// Weights and KV caches stay in the caller's memory (tensors point at it); each step
// builds the executor's graph for (s, n_kv), allocates its intermediates with
// ggml-alloc and runs ggml_graph_compute on n_threads.
//
// Per layer (gamma of RMSNorm baked into the following Linear, Q/K/V and gate/up
// fused, as ggmlc's fusion pass emits them):
//   h = rms_norm(x); qkv = mul_mat(Wqkv, h); q, k = rope_ext(NEOX)(views of qkv)
//   set_rows(Kc, k^T, idx); set_rows(Vc, v^T, idx)          (executor.cpp:2181-2184)
//   a = flash_attn_ext(q^T, Kc[:n_kv], Vc[:n_kv], mask, 1/sqrt(hd))  (:2195-2197)
//   x += mul_mat(Wo, a); x += mul_mat(Wdown, swiglu(mul_mat(Wgate_up, rms_norm(x))))
// then rms_norm(x[s-1]) -> mul_mat(lm_head) -> argmax. A projection with a bias
// (ref_llama_set_bias) is ggml_add(mul_mat(W, h), b), the executor's MUL_MAT with a third
// input (executor.cpp:2436-2445).

struct RefLlama {
    int64_t n_layer, n_embd, n_head, n_head_kv, hd, n_ff, n_vocab, max_ctx;
    ggml_type wt;
    float eps, base;
    ggml_context* wctx = nullptr;
    ggml_tensor *embed = nullptr, *lm_head = nullptr;
    std::vector<ggml_tensor*> wqkv, wo, wgu, wd, kc, vc;
    std::vector<ggml_tensor*> bias;  // [4 * layer + which] or null
    ggml_gallocr_t galloc = nullptr;
    std::vector<uint8_t> work;
};

static ggml_tensor* ext2d(ggml_context* c, ggml_type t, int64_t ne0, int64_t ne1, const void* p) {
    ggml_tensor* x = ggml_new_tensor_2d(c, t, ne0, ne1);
    x->data = const_cast<void*>(p);
    return x;
}

// dims: n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, max_ctx
// layer_w: 4 pointers per layer (qkv, o, gate_up, down); kv: 2 per layer (K, V caches,
// F16 [max_ctx][hd] per head, heads outermost)
void* ref_llama_create(const int64_t* dims, int wtype, float eps, float rope_base, const void* embed,
                       const void* lm_head, const void* const* layer_w, void* const* kv) {
    ggml_cpu_init();
    RefLlama* m = new RefLlama;
    m->n_layer = dims[0], m->n_embd = dims[1], m->n_head = dims[2], m->n_head_kv = dims[3];
    m->hd = dims[4], m->n_ff = dims[5], m->n_vocab = dims[6], m->max_ctx = dims[7];
    m->wt = (ggml_type)wtype, m->eps = eps, m->base = rope_base;
    ggml_init_params p = {ggml_tensor_overhead() * (size_t)(12 * m->n_layer + 8), nullptr, true};
    m->wctx = ggml_init(p);
    if (!m->wctx) {
        delete m;
        return nullptr;
    }
    const int64_t E = m->n_embd, qd = m->n_head * m->hd, kvd = m->n_head_kv * m->hd;
    m->embed = ext2d(m->wctx, m->wt, E, m->n_vocab, embed);
    m->lm_head = ext2d(m->wctx, m->wt, E, m->n_vocab, lm_head);
    for (int64_t l = 0; l < m->n_layer; ++l) {
        m->wqkv.push_back(ext2d(m->wctx, m->wt, E, qd + 2 * kvd, layer_w[4 * l + 0]));
        m->wo.push_back(ext2d(m->wctx, m->wt, qd, E, layer_w[4 * l + 1]));
        m->wgu.push_back(ext2d(m->wctx, m->wt, E, 2 * m->n_ff, layer_w[4 * l + 2]));
        m->wd.push_back(ext2d(m->wctx, m->wt, m->n_ff, E, layer_w[4 * l + 3]));
        for (int j = 0; j < 2; ++j) {
            ggml_tensor* c = ggml_new_tensor_4d(m->wctx, GGML_TYPE_F16, m->hd, m->max_ctx, m->n_head_kv, 1);
            c->data = kv[2 * l + j];
            (j ? m->vc : m->kc).push_back(c);
        }
    }
    m->bias.assign(4 * m->n_layer, nullptr);
    m->galloc = ggml_gallocr_new(ggml_backend_cpu_buffer_type());
    return m;
}

// bias of layer l's projection `which` (0 qkv, 1 o, 2 gate_up, 3 down): F32 [N] in the
// caller's memory, N = that projection's output rows. Returns 0 on success.
int ref_llama_set_bias(void* h, int64_t l, int which, const float* b, int64_t n) {
    RefLlama* m = (RefLlama*)h;
    if (!m || l < 0 || l >= m->n_layer || which < 0 || which > 3) return -1;
    const ggml_tensor* w = which == 0 ? m->wqkv[l] : which == 1 ? m->wo[l] : which == 2 ? m->wgu[l] : m->wd[l];
    if (n != w->ne[1]) return -1;
    ggml_tensor* t = ggml_new_tensor_1d(m->wctx, GGML_TYPE_F32, n);
    t->data = const_cast<float*>(b);
    m->bias[4 * l + which] = t;
    return 0;
}

// the executor's MUL_MAT node: mul_mat(W, x), + bias when the node has one
static ggml_tensor* linear(ggml_context* c, ggml_tensor* w, ggml_tensor* x, ggml_tensor* b) {
    ggml_tensor* r = ggml_mul_mat(c, w, x);
    return b ? ggml_add(c, r, b) : r;
}

// ids I32 [s]; mask F16 [s][n_kv] (row i = query pos+i); logits F32 [n_vocab] of the
// last token; next = its argmax. Returns 0 on success.
int ref_llama_step(void* h, const int32_t* ids, int64_t s, int64_t pos, int64_t n_kv, const uint16_t* mask,
                   float* logits, int32_t* next, int n_threads) {
    RefLlama* m = (RefLlama*)h;
    if (pos + s > m->max_ctx || n_kv > m->max_ctx || pos + s > n_kv) return -1;
    const size_t graph_size = 64 * (size_t)m->n_layer + 64;
    ggml_init_params p = {ggml_tensor_overhead() * graph_size * 2 + ggml_graph_overhead_custom(graph_size, false),
                          nullptr, true};
    ggml_context* c = ggml_init(p);
    if (!c) return -1;
    ggml_cgraph* gf = ggml_new_graph_custom(c, graph_size, false);
    const int64_t E = m->n_embd, hd = m->hd, H = m->n_head, Hk = m->n_head_kv;
    const int64_t qd = H * hd, kvd = Hk * hd;

    ggml_tensor* t_ids = ggml_new_tensor_1d(c, GGML_TYPE_I32, s);
    ggml_tensor* t_pos = ggml_new_tensor_1d(c, GGML_TYPE_I32, s);
    ggml_tensor* t_idx = ggml_new_tensor_1d(c, GGML_TYPE_I64, s);
    ggml_tensor* t_mask = ggml_new_tensor_2d(c, GGML_TYPE_F16, n_kv, s);
    for (ggml_tensor* t : {t_ids, t_pos, t_idx, t_mask}) ggml_set_input(t);

    ggml_tensor* x = ggml_get_rows(c, m->embed, t_ids);  // [E, s]
    const float scale = 1.0f / sqrtf((float)hd);
    for (int64_t l = 0; l < m->n_layer; ++l) {
        ggml_tensor* hn = ggml_rms_norm(c, x, m->eps);
        ggml_tensor* qkv = linear(c, m->wqkv[l], hn, m->bias[4 * l]);  // [qd + 2 kvd, s]
        const size_t es = sizeof(float);
        ggml_tensor* q = ggml_view_3d(c, qkv, hd, H, s, hd * es, qkv->nb[1], 0);
        ggml_tensor* k = ggml_view_3d(c, qkv, hd, Hk, s, hd * es, qkv->nb[1], qd * es);
        ggml_tensor* v = ggml_view_3d(c, qkv, hd, Hk, s, hd * es, qkv->nb[1], (qd + kvd) * es);
        q = ggml_rope_ext(c, q, t_pos, nullptr, (int)hd, GGML_ROPE_TYPE_NEOX, 0, m->base, 1.0f, 0.0f, 1.0f,
                          0.0f, 0.0f);
        k = ggml_rope_ext(c, k, t_pos, nullptr, (int)hd, GGML_ROPE_TYPE_NEOX, 0, m->base, 1.0f, 0.0f, 1.0f,
                          0.0f, 0.0f);
        // [hd, heads, s] -> [hd, s, heads] (rows stay contiguous, as set_rows requires)
        ggml_tensor* ks = ggml_permute(c, k, 0, 2, 1, 3);
        ggml_tensor* vs = ggml_permute(c, v, 0, 2, 1, 3);
        ggml_build_forward_expand(gf, ggml_set_rows(c, m->kc[l], ks, t_idx));
        ggml_build_forward_expand(gf, ggml_set_rows(c, m->vc[l], vs, t_idx));
        ggml_tensor* K = ggml_view_4d(c, m->kc[l], hd, n_kv, Hk, 1, m->kc[l]->nb[1], m->kc[l]->nb[2],
                                      m->kc[l]->nb[3], 0);
        ggml_tensor* V = ggml_view_4d(c, m->vc[l], hd, n_kv, Hk, 1, m->vc[l]->nb[1], m->vc[l]->nb[2],
                                      m->vc[l]->nb[3], 0);
        ggml_tensor* a = ggml_flash_attn_ext(c, ggml_permute(c, q, 0, 2, 1, 3), K, V, t_mask, scale, 0.0f, 0.0f);
        a = ggml_reshape_2d(c, a, qd, s);  // the op's output is [hd, H, s]
        x = ggml_add(c, x, linear(c, m->wo[l], a, m->bias[4 * l + 1]));
        ggml_tensor* gu = linear(c, m->wgu[l], ggml_rms_norm(c, x, m->eps), m->bias[4 * l + 2]);
        x = ggml_add(c, x, linear(c, m->wd[l], ggml_swiglu(c, gu), m->bias[4 * l + 3]));
    }
    ggml_tensor* xl = ggml_view_2d(c, x, E, 1, x->nb[1], (size_t)(s - 1) * x->nb[1]);
    ggml_tensor* lo = ggml_mul_mat(c, m->lm_head, ggml_rms_norm(c, xl, m->eps));
    ggml_tensor* am = ggml_argmax(c, lo);
    ggml_set_output(lo);
    ggml_set_output(am);
    ggml_build_forward_expand(gf, am);

    int rc = -1;
    if (ggml_gallocr_alloc_graph(m->galloc, gf)) {
        memcpy(t_ids->data, ids, sizeof(int32_t) * s);
        int32_t* pp = (int32_t*)t_pos->data;
        int64_t* ip = (int64_t*)t_idx->data;
        for (int64_t i = 0; i < s; ++i) pp[i] = (int32_t)(pos + i), ip[i] = pos + i;
        memcpy(t_mask->data, mask, sizeof(uint16_t) * n_kv * s);
        ggml_cplan plan = ggml_graph_plan(gf, n_threads, nullptr);
        if (m->work.size() < plan.work_size) m->work.resize(plan.work_size);
        plan.work_data = m->work.data();
        if (ggml_graph_compute(gf, &plan) == GGML_STATUS_SUCCESS) {
            memcpy(logits, lo->data, sizeof(float) * m->n_vocab);
            *next = *(const int32_t*)am->data;
            rc = 0;
        }
    }
    ggml_free(c);
    return rc;
}

void ref_llama_free(void* h) {
    RefLlama* m = (RefLlama*)h;
    if (!m) return;
    if (m->galloc) ggml_gallocr_free(m->galloc);
    ggml_free(m->wctx);
    delete m;
}

}  // extern "C"
