// FLASH_ATTN_EXT over an F16 KV cache view (decode and chunked prefill).
//
// Semantics: ggml_compute_forward_flash_attn_ext_f16 (ggml-cpu/ops.cpp:
// 8532-8768 one_chunk, 8770-9058 tiled, 9060-9209 split-KV decode): per query
// row i and head h, with kv head h / (Hq / Hkv) (GQA broadcast, rk2),
//   s_j = scale * q . k_j (softcap: c * tanh(s / c)) + slope_h * mask[i, j]
//   out = sum_j exp(s_j - max) v_j / sum_j exp(s_j - max),
// written to dst[i][h][:] (the op's permute(0, 2, 1, 3)). The query is rounded
// to fp16 for S < 64 (one_chunk converts it to the K type) and kept fp32 for
// S >= 64 (tiled path); everything is accumulated in fp32, which is closer to
// the exact softmax than the CPU's fp16 V accumulator (ops.cpp:8682-8696).
//
// Split-KV ("flash decoding"): the KV range is cut into 64-row chunks;
// a workgroup owns (split, kv head, tile of 16 query vectors) — the query
// vectors of one kv head are the G = Hq/Hkv heads x S rows that share it, so
// every K/V byte is read once per tile. Each workgroup streams its chunks
// through LDS with an online softmax; when the KV range is split across
// workgroups, unnormalised partials (O, max, sum) go to the workspace and a
// second kernel merges them (the reduction of ops.cpp:9060-9128).
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace gq {

namespace {

constexpr int CH = 64;   // kv rows per chunk
constexpr int QT = 16;   // query vectors per tile
constexpr int TARGET_WG = 1024;

constexpr int DEC_MAX_NQ = 8;     // query vectors per kv head served by the decode kernel
constexpr int DEC_TARGET_WG = 512;
constexpr int MAX_SPLIT = 1024;

// Fused split merge of the decode kernel: the last workgroup to finish a (sequence,
// kv head) merges that pair's split partials itself, so no second launch is needed.
// Partials are written and read with agent-scope relaxed atomics (coherent across the
// XCDs' L2s, no cache flushes) and each workgroup arrives on the pair's counter after
// its own stores have completed. A launch needs its counters at zero and leaves them at
// zero (the last arrival resets its counter). The counters are not in the caller's
// workspace: that holds whatever the previous op left there, and clearing it would cost
// a launch. Instead each stream gets a set of its own (ARRIVE_SETS sets, assigned on a
// stream's first fused launch; launches on one stream never overlap), so launches on
// different streams cannot collide; a stream past the last set takes the separate merge
// launch. Launches captured in a graph keep their stream's set, so two graphs captured
// on one stream must not be replayed concurrently.
constexpr int ARRIVE_N = 4096;     // (sequence, kv head) pairs of one launch
constexpr int ARRIVE_SETS = 16;    // streams with counters of their own
constexpr int FUSE_MAX_SPLIT = 16;  // splits merged from registers (one round trip)
__device__ unsigned g_attn_arrive[ARRIVE_SETS * ARRIVE_N];

// Per-wave timestamps of k_attn_dec (s_memrealtime, 100 MHz), compiled only into the
// benchmark's measurement library (GQ_ATTN_STAMPS; libgq has none of this): event e of
// wave w of workgroup (x, y) at g_attn_stamps[((y * gridDim.x + x) * 4 + w) * 8 + e];
// 0 start, 1 K/V loads issued and the query scaled, 2 first K row converted, 3 every row
// scored and accumulated, 4 partial stored, 5 arrival counted, 6 merge written, 7 end (0:
// not reached). Stamps 2 and 3 take a register of the data as an asm input, so they cannot
// be read before the loads they follow have returned.
#ifdef GQ_ATTN_STAMPS
constexpr int STAMP_SLOTS = 4096 * 4 * 8;
__device__ unsigned long long g_attn_stamps[STAMP_SLOTS];
#define GQ_STAMP(e)                                           \
    do {                                                      \
        __builtin_amdgcn_sched_barrier(0);                    \
        stamp_[e] = __builtin_amdgcn_s_memrealtime();         \
        __builtin_amdgcn_sched_barrier(0);                    \
    } while (0)
#define GQ_STAMP_AFTER(e, x)                                                           \
    do {                                                                               \
        unsigned long long t_;                                                         \
        asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t_) : "v"(x)); \
        stamp_[e] = t_;                                                                \
    } while (0)
#define GQ_STAMP_FLUSH()                                                                                 \
    do {                                                                                                 \
        GQ_STAMP(7);                                                                                     \
        const size_t i_ = (((size_t)blockIdx.y * gridDim.x + blockIdx.x) * 4 + (threadIdx.x >> 6)) * 8; \
        if ((threadIdx.x & 63) == 0 && i_ + 8 <= (size_t)STAMP_SLOTS)                                    \
            for (int e_ = 0; e_ < 8; ++e_) g_attn_stamps[i_ + e_] = stamp_[e_];                          \
    } while (0)
#else
#define GQ_STAMP(e) \
    do {            \
    } while (0)
#define GQ_STAMP_AFTER(e, x) \
    do {                     \
    } while (0)
#define GQ_STAMP_FLUSH() \
    do {                 \
    } while (0)
#endif

// the counter set of a stream (its first fused launch assigns one), or -1 when every set
// is taken
int arrive_set(hipStream_t s) {
    static std::mutex mu;
    static hipStream_t owner[ARRIVE_SETS];
    static int used = 0;
    std::lock_guard<std::mutex> lk(mu);
    for (int i = 0; i < used; ++i)
        if (owner[i] == s) return i;
    if (used == ARRIVE_SETS) return -1;
    owner[used] = s;
    return used++;
}

__device__ __forceinline__ void st_ag(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_ag(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Arrive once this workgroup's partial stores are complete; true in the last arrival of
// the pair (which also resets the pair's counter to zero). Every thread of the workgroup
// calls it.
// What this relies on (gfx950, as on gfx942): agent-scope atomic stores and loads carry
// the sc1 bit, so they bypass the per-XCD L2 for coherence and are served by memory
// (through the Infinity Fabric / MALL), never by a stale L2 line of another XCD;
// s_waitcnt vmcnt(0) returns only after every such store has been acknowledged at that
// level; the counter's fetch_add is performed at the same level, so a workgroup that
// reads n_split - 1 from it runs after every other workgroup's partials are visible to
// sc1 loads. The loads of the merge are atomic, so the compiler cannot hoist them above
// the __syncthreads that follows the arrival. The C++/HIP memory model would ask for a
// release fetch_add and an acquire fence instead; both write back / invalidate the whole
// XCD L2 on this target (measured: the merge took 38 us instead of ~2 us), so the
// protocol stays at the hardware level. gq_attn_reset_counters clears the counters
// after a launch that did not finish.
__device__ __forceinline__ bool arrive_last(unsigned* ctr, int n_split) {
    __shared__ int sLast;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = old == (unsigned)(n_split - 1);
        if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sLast = last;
    }
    __syncthreads();
    return sLast != 0;
}

// The reduction of k_attn_merge for one (query vector, dim d) with the same operations in
// the same order, every split's (m, l, o) requested at once: one memory round trip
// (n_split <= FUSE_MAX_SPLIT). base: split 0's partial row; stride: floats between splits.
__device__ __forceinline__ float merge_splits_ag(const float* base, int64_t stride, int n_split, int d);

struct Plan {
    int64_t G, NQ, n_qt, n_chunks, cps, n_split;
    bool dec;               // k_attn_dec: one workgroup per (split, kv head), all NQ queries
    int64_t rows_per_split;  // dec only
    int dec_u;               // dec only: rows per lane stream
};

// the split merge runs inside the decode kernel when one thread per (query vector,
// dim) can hold every split's partial in registers and the launch's (sequence, kv
// head) pairs fit the counters, unless GQ_OPT_ATTN_SEPARATE_MERGE asks for the
// second launch (comparison runs; the results are the same bits)
bool fuse_merge_ok(int64_t n_split, int64_t nq, int64_t D, int64_t pairs) {
    return !option_attn_separate_merge() && n_split > 1 && n_split <= FUSE_MAX_SPLIT && nq * D <= 256 &&
           pairs <= ARRIVE_N;
}

// the kernels' head-dim width: 64, 128 or 256 (other head dims, multiples of 8, are padded:
// their loads past the head read 0 and nothing past it is stored)
int64_t attn_width(int64_t D) { return D <= 64 ? 64 : (D <= 128 ? 128 : 256); }

Plan make_plan(int64_t D, int64_t S, int64_t Hq, int64_t Hkv, int64_t n_kv) {
    Plan p;
    p.G = Hq / Hkv;
    p.NQ = p.G * S;
    p.n_qt = cdiv(p.NQ, QT);
    p.n_chunks = cdiv(n_kv, CH);
    p.dec = p.NQ <= DEC_MAX_NQ;
    if (p.dec) {
        // rows per split = U rows per lane stream x (4 waves x rows per wave instruction);
        // the largest U (8, 4, 2; at most 4 for more than 4 query vectors) that still
        // gives DEC_TARGET_WG / 2 workgroups
        const int64_t rows_it = 4 * (64 / (attn_width(D) / 8));
        const int umax = p.NQ > 4 ? 4 : 8;
        int u = umax;
        while (u > 2 && Hkv * cdiv(n_kv, u * rows_it) < DEC_TARGET_WG / 2) u >>= 1;
        // one query vector per kv head (MHA decode), 128-dim: 160- or 192-row splits when
        // they need fewer rounds of workgroups over the CUs (rounds x rows per split), so a
        // 32-head launch at n_kv = 1280 is one workgroup per CU (measured: tg128 +0.65%)
        if (p.NQ == 1 && D == 128 && u == 8) {
            const int64_t ncu = 256;
            int64_t best = cdiv(Hkv * cdiv(n_kv, 8 * rows_it), ncu) * 8;
            for (int c : {10, 12}) {
                const int64_t ns = cdiv(n_kv, c * rows_it);
                const int64_t cost = cdiv(Hkv * ns, ncu) * c;
                if (ns <= FUSE_MAX_SPLIT && cost < best) best = cost, u = c;
            }
        }
        p.dec_u = u;
        p.rows_per_split = u * rows_it;
        p.n_split = cdiv(n_kv, p.rows_per_split);
        p.cps = 0;
        // the merge holds one weight per split in LDS: longer contexts take the tiled kernel
        if (p.n_split <= MAX_SPLIT) return p;
        p.dec = false;
        p.dec_u = 0;
    }
    const int64_t base = Hkv * p.n_qt;
    int64_t want = base >= TARGET_WG ? 1 : cdiv(TARGET_WG, base);
    if (want > p.n_chunks) want = p.n_chunks;
    if (want < 1) want = 1;
    p.cps = cdiv(p.n_chunks, want);
    p.n_split = cdiv(p.n_chunks, p.cps);
    p.rows_per_split = 0;
    return p;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// sum over aligned groups of W lanes (W = 8, 16 or 32) with DPP (and a permlane swap of
// the 16-lane totals for 32); every lane gets its group's total
__device__ __forceinline__ float add_16(float x);
template <int W>
__device__ __forceinline__ float lanes_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror: 8-lane totals
    if constexpr (W >= 16) v += dpp_f<0x140>(v);  // row_mirror: 16-lane totals
    if constexpr (W == 32) v = add_16(v);         // 32-lane totals
    return v;
}

// value pairs {own, partner} for partner = lane ^ 8 (within rows of 16), lane ^ 16, lane ^ 32
struct Pair {
    float a, b;
};
__device__ __forceinline__ Pair xchg_row8(float x) { return {x, dpp_f<0x128>(x)}; }  // row_ror:8
__device__ __forceinline__ Pair xchg_16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ Pair xchg_32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ float add_16(float x) {  // x + the value of lane ^ 16 (same bits in both)
    const Pair p = xchg_16(x);
    return p.a + p.b;
}

// online-softmax states (m, l, o[8]) of two lanes merged into both
template <typename X>
__device__ __forceinline__ void merge_pair(float& m, float& l, float (&o)[8], X xchg) {
    const Pair pm = xchg(m), pl = xchg(l);
    const float mn = fmaxf(pm.a, pm.b);
    const float a1 = mn == -INFINITY ? 0.0f : __expf(pm.a - mn);
    const float a2 = mn == -INFINITY ? 0.0f : __expf(pm.b - mn);
    l = pl.a * a1 + pl.b * a2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const Pair po = xchg(o[e]);
        o[e] = po.a * a1 + po.b * a2;
    }
    m = mn;
}

__device__ __forceinline__ void h8_to_f(const uint4 w, float* f) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        f[2 * e] = h2f((uint16_t)(u[e] & 0xffff));
        f[2 * e + 1] = h2f((uint16_t)(u[e] >> 16));
    }
}

// Decode attention: few query vectors per kv head (G*S <= 8). A workgroup owns
// (split, kv head) and rows [split*rps, (split+1)*rps) of the KV view. Each
// wave instruction reads 64/(D/8) whole K (or V) rows, 16 bytes per lane, so
// every lane group of D/8 lanes is a row stream with its own online-softmax
// state (m, l, o[8 dims] per query); rows whose mask is -inf for every query
// are not read. Streams merge by shuffles inside the wave and through LDS across
// the 4 waves; the result is the output (one split) or an fp32 partial
// (O, max, sum) for k_attn_merge.
//
// PAGED (batched decode over a paged KV pool): blockIdx.z is the sequence b, whose
// query vectors are row b of q (the G heads of this kv head) and whose logical KV
// rows [0, len_b) live in pages of P rows: logical row r is pool row
// table[b][r / P] * P + r % P. A split never crosses a page (P % rps == 0), so one
// table entry per workgroup locates all its rows; rows past len_b (and splits past
// it, or with a negative page id) read nothing and weigh 0. Partials are indexed by
// query vector b * G + u, so k_attn_merge finishes them as B * G query rows.
// qmode: bit 0 rounds the query to fp16 (the CPU decode path), bit 1 says its rows are
// 16-byte aligned (two 16-byte loads per lane instead of eight 4-byte ones).
template <int D, int NQ, int U, bool PAGED>
__global__ __launch_bounds__(256) void k_attn_dec(AttnArgs a, int G, int nq, int64_t rps, int n_split, float m0,
                                                  float m1, uint32_t n_head_log2, int qmode,
                                                  float* __restrict__ part, PagedKv pg, int fuse) {
    // fuse: 0 separate merge, else 1 + the stream's counter set (arrive_set)
#ifdef GQ_ATTN_STAMPS
    unsigned long long stamp_[8] = {};
#endif
    GQ_STAMP(0);
    constexpr int LPR = D / 8;       // lanes per row
    constexpr int RPI = 64 / LPR;    // rows per wave instruction
    constexpr int ROWS_IT = 4 * RPI;
    __shared__ float sM[4][NQ], sL[4][NQ];
    __shared__ __align__(16) float sO[4][NQ][D];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane / LPR, d0 = (lane % LPR) * 8;
    const int split = blockIdx.x, hk = blockIdx.y;
    const int Hkv = (int)a.Hkv;
    const int seq = PAGED ? (int)blockIdx.z : 0;
    int64_t r_begin = (int64_t)split * rps, r_len = a.n_kv, prow0 = r_begin;
    if constexpr (PAGED) {
        r_len = pg.len[seq];
        const int64_t pi = r_begin >> pg.log2p;
        const int page = (r_begin < r_len && pi < pg.tstride) ? pg.table[seq * pg.tstride + pi] : -1;
        if (page < 0) r_len = 0;  // nothing to read for this split
        prow0 = ((int64_t)(page < 0 ? 0 : page) << pg.log2p) + (r_begin & ((1 << pg.log2p) - 1));
    }

    float q[NQ][8], slope[NQ];
    const uint16_t* mrow[NQ];
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
        const int uu = u < nq ? u : 0;
        const int64_t h = (int64_t)hk * G + uu % G, i = seq + uu / G;
        const float* qp = reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(a.q) + i * a.qnb1 +
                                                         h * a.qnb2) + d0;
        if ((qmode & 2) && d0 < a.D) {  // 16-byte aligned q rows: two 16-byte loads
            const float4 x0 = *reinterpret_cast<const float4*>(qp);
            const float4 x1 = *reinterpret_cast<const float4*>(qp + 4);
            q[u][0] = x0.x, q[u][1] = x0.y, q[u][2] = x0.z, q[u][3] = x0.w;
            q[u][4] = x1.x, q[u][5] = x1.y, q[u][6] = x1.z, q[u][7] = x1.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) q[u][e] = d0 < a.D ? qp[e] : 0.0f;  // dims past a.D: 0
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if (qmode & 1) q[u][e] = (float)(_Float16)q[u][e];
            q[u][e] *= a.scale;  // folded: (q*scale).k, the order ggml's tiled path uses is irrelevant at 1e-6
        }
        slope[u] = 1.0f;
        if (a.max_bias > 0.0f)
            slope[u] = h < n_head_log2 ? powf(m0, (float)(h + 1)) : powf(m1, (float)(2 * (h - n_head_log2) + 1));
        mrow[u] = a.mask ? reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(a.mask) + i * a.mnb1)
                         : nullptr;
    }

    float m[NQ], l[NQ], o[NQ][8];
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
        m[u] = -INFINITY, l[u] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[u][e] = 0.0f;
    }

    const int64_t r_end = min<int64_t>(r_len, r_begin + rps);

    // All U rows of this lane's stream (rows r0 + t * ROWS_IT) are requested at once,
    // together with their mask values: one memory round trip per workgroup. K/V rows
    // are raw buffer loads over [0, n_kv) of this head, so rows past n_kv return 0
    // without a fetch; masked rows are read and then weigh exp(-inf) = 0.
    const int64_t r0 = r_begin + wave * RPI + grp;
    auto rsrc = [&](const void* p, int64_t nb2, int64_t nb1) {
        const uint64_t base = reinterpret_cast<uint64_t>(p) + (uint64_t)(hk * nb2);
        const int64_t bytes = a.n_kv * nb1;
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
        const uint32_t n = (uint32_t)(bytes > 0x7fffffff ? 0x7fffffff : bytes);
        return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                                 (int)__builtin_amdgcn_readfirstlane(n), 0x00020000);
    };
    const __amdgpu_buffer_rsrc_t krs = rsrc(a.k, a.knb2, a.knb1), vrs = rsrc(a.v, a.vnb2, a.vnb1);
    // mask rows as buffers too (no mask: an empty resource, every value reads 0)
    __amdgpu_buffer_rsrc_t mrs[NQ];
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
        const uint64_t base = reinterpret_cast<uint64_t>(mrow[u]);
        const uint32_t n = mrow[u] ? (uint32_t)(r_len * 2 > 0x7fffffff ? 0x7fffffff : r_len * 2) : 0u;
        // readfirstlane returns int: both halves go through uint32_t so the low half is
        // zero-extended when the address is put back together
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
        mrs[u] = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                                   (int)__builtin_amdgcn_readfirstlane(n), 0x00020000);
    }
    u32x4 kw[U], vw[U];
    uint16_t mb[U][NQ];
    bool rin[U];
#pragma unroll
    for (int t = 0; t < U; ++t) {
        const int64_t r = r0 + (int64_t)t * ROWS_IT;
        const bool in = r < r_end;
        rin[t] = in;
        const int64_t pr = prow0 + (r - r_begin);  // pool row (the row itself when not paged)
        const bool dim_in = d0 < a.D;  // head dims padded to the template's D read 0
        const uint32_t ko = in && dim_in ? (uint32_t)(pr * a.knb1 + d0 * 2) : 0x80000000u;
        const uint32_t vo = in && dim_in ? (uint32_t)(pr * a.vnb1 + d0 * 2) : 0x80000000u;
        kw[t] = __builtin_amdgcn_raw_buffer_load_b128(krs, (int)ko, 0, 0);
        vw[t] = __builtin_amdgcn_raw_buffer_load_b128(vrs, (int)vo, 0, 0);
#pragma unroll
        for (int u = 0; u < NQ; ++u)
            mb[t][u] = __builtin_amdgcn_raw_buffer_load_b16(mrs[u], in ? (int)(r * 2) : (int)0x80000000, 0, 0);
    }
    // the mask values are converted only once every row's loads are in flight (a use
    // right after its load would wait for all loads issued before it)
    __builtin_amdgcn_sched_barrier(0);
    GQ_STAMP(1);
    float mk[U][NQ];
#pragma unroll
    for (int t = 0; t < U; ++t) {
#pragma unroll
        for (int u = 0; u < NQ; ++u) {
            const float x = h2f(mb[t][u]);
            mk[t][u] = !rin[t] || u >= nq ? -INFINITY : (x == -INFINITY ? -INFINITY : slope[u] * x);
        }
    }
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
        float sc[U];
        float mx = m[u];
#pragma unroll
        for (int t = 0; t < U; ++t) {
            float kf[8];
            h8_to_f(make_uint4(kw[t].x, kw[t].y, kw[t].z, kw[t].w), kf);
#ifdef GQ_ATTN_STAMPS
            if (u == 0 && t == 0) GQ_STAMP_AFTER(2, kf[0]);
#endif
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc = fmaf(q[u][e], kf[e], acc);
            acc = lanes_sum<LPR>(acc);
            if (a.softcap != 0.0f) acc = a.softcap * tanhf(acc);
            sc[t] = mk[t][u] == -INFINITY ? -INFINITY : acc + mk[t][u];
            mx = fmaxf(mx, sc[t]);
        }
        if (mx == -INFINITY) continue;
        const float al = __expf(m[u] - mx);  // exp(-inf) = 0 for an empty stream
        l[u] *= al;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[u][e] *= al;
#pragma unroll
        for (int t = 0; t < U; ++t) {
            const float p = __expf(sc[t] - mx);
            float vf[8];
            h8_to_f(make_uint4(vw[t].x, vw[t].y, vw[t].z, vw[t].w), vf);
            l[u] += p;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[u][e] = fmaf(p, vf[e], o[u][e]);
        }
        m[u] = mx;
    }

    GQ_STAMP_AFTER(3, o[0][0]);
    // merge the row streams of the wave: partner lanes (xor 8 for D = 64, then xor 16,
    // xor 32) exchanged with DPP / permlane swaps (VALU, no LDS); the merge of two
    // (m, l, o) states is symmetric, so each lane may combine the pair in any order
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
        if constexpr (LPR == 8) merge_pair(m[u], l[u], o[u], xchg_row8);
        if constexpr (LPR <= 16) merge_pair(m[u], l[u], o[u], xchg_16);
        merge_pair(m[u], l[u], o[u], xchg_32);
    }
    if (grp == 0) {
#pragma unroll
        for (int u = 0; u < NQ; ++u) {
            *reinterpret_cast<float4*>(&sO[wave][u][d0]) = make_float4(o[u][0], o[u][1], o[u][2], o[u][3]);
            *reinterpret_cast<float4*>(&sO[wave][u][d0 + 4]) = make_float4(o[u][4], o[u][5], o[u][6], o[u][7]);
            if (lane == 0) sM[wave][u] = m[u], sL[wave][u] = l[u];
        }
    }
    __syncthreads();
    // merge the 4 waves and write
    for (int idx = tid; idx < nq * D; idx += 256) {
        const int u = idx / D, d = idx % D;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) mx = fmaxf(mx, sM[w][u]);
        float L = 0.0f, acc = 0.0f;
        if (mx != -INFINITY) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float f = __expf(sM[w][u] - mx);
                L += sL[w][u] * f;
                acc += sO[w][u][d] * f;
            }
        }
        const int64_t h = (int64_t)hk * G + u % G, i = seq + u / G;
        if (n_split == 1) {
            if (d < a.D) a.dst[(i * a.Hq + h) * a.D + d] = L == 0.0f ? 0.0f : acc / L;
        } else {
            const int64_t nqt = PAGED ? (int64_t)pg.B * nq : nq;  // query vectors of all sequences
            float* pp = part + (((int64_t)split * Hkv + hk) * nqt + (int64_t)seq * nq + u) * (D + 2);
            if (fuse) {
                st_ag(pp + 2 + d, acc);
                if (d == 0) st_ag(pp, mx), st_ag(pp + 1, L);
            } else {
                pp[2 + d] = acc;
                if (d == 0) pp[0] = mx, pp[1] = L;
            }
        }
    }
    GQ_STAMP(4);
    if (!fuse || n_split == 1) {
        GQ_STAMP_FLUSH();
        return;
    }
    const bool last = arrive_last(&g_attn_arrive[(fuse - 1) * ARRIVE_N + seq * Hkv + hk], n_split);
    GQ_STAMP(5);
    if (!last) {
        GQ_STAMP_FLUSH();
        return;
    }
    const int u = tid / D, d = tid % D;  // one thread per (query vector, dim): nq <= 256 / D
    if (u < nq) {
        const int64_t nqt = PAGED ? (int64_t)pg.B * nq : nq;
        const float mo = merge_splits_ag(part + ((int64_t)hk * nqt + (int64_t)seq * nq + u) * (D + 2),
                                         (int64_t)Hkv * nqt * (D + 2), n_split, d);
        const int64_t h = (int64_t)hk * G + u % G, i = seq + u / G;
        if (d < a.D) a.dst[(i * a.Hq + h) * a.D + d] = mo;
    }
    GQ_STAMP(6);
    GQ_STAMP_FLUSH();
}

__device__ __forceinline__ float merge_splits_ag(const float* base, int64_t stride, int n_split, int d) {
    float pm[FUSE_MAX_SPLIT], pl[FUSE_MAX_SPLIT], po[FUSE_MAX_SPLIT];
#pragma unroll
    for (int s2 = 0; s2 < FUSE_MAX_SPLIT; ++s2) {
        if (s2 < n_split) {
            pm[s2] = ld_ag(base + s2 * stride);
            pl[s2] = ld_ag(base + s2 * stride + 1);
            po[s2] = ld_ag(base + s2 * stride + 2 + d);
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int s2 = 0; s2 < FUSE_MAX_SPLIT; ++s2) {
        if (s2 < n_split) {
            pm[s2] = pl[s2] == 0.0f ? -INFINITY : pm[s2];
            mx = fmaxf(mx, pm[s2]);
        }
    }
    float L = 0.0f, acc = 0.0f;
#pragma unroll
    for (int s2 = 0; s2 < FUSE_MAX_SPLIT; ++s2) {
        if (s2 < n_split) {
            const float w = pm[s2] == -INFINITY ? 0.0f : __expf(pm[s2] - mx);
            L += pl[s2] * w;
            acc += po[s2] * w;
        }
    }
    return L == 0.0f ? 0.0f : acc / L;
}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// Prefill attention on the matrix cores (v_mfma_f32_16x16x32_f16), no ALiBi / softcap.
// A workgroup owns 16 WQ query vectors of one kv head (WQ waves x 16), walks the KV range
// in blocks of 64 keys staged in LDS (K as [key][dim], V transposed to [dim][key]),
// and keeps an online softmax per query in registers:
//   S^T (16 keys x 16 queries tiles) = K_blk . Q^T, with Q = q_hi + q_lo split into two
//   fp16 parts (q_lo = 0 when the query is rounded to fp16), so the scores carry fp32
//   accuracy; s = S * scale + mask; O^T += V^T . P^T with P = p_hi + p_lo split the same
//   way (fp32-level products, accumulated in fp32).
// MFMA 16x16x32 operand layouts (lane l, j = l % 16, g = l / 16): A[i][k]: i = j,
// k = 8g..8g+7; B[k][n]: n = j, k = 8g..8g+7; C[i][n]: n = j, i = 4g..4g+3. The
// S^T accumulator of lane l therefore holds query j and keys 16t + 4g + r; used as the
// B operand of the PV product (K = 32 keys of tiles t0, t1) its 8 values are keys
// (4g..4g+3, 16+4g..16+4g+3), and the V^T operand is read in that same key order.
template <int D, int WQ = 4>
__global__ __launch_bounds__(64 * WQ) void k_attn_mma(AttnArgs a, int G, int NQ, int q_f16) {
    static_assert(WQ == 2 || WQ == 4, "2 or 4 waves of 16 query vectors");
    constexpr int BKV = 64;
    constexpr int LDK = D + 8;      // halves per K row in LDS
    constexpr int LDV = BKV + 8;    // halves per V^T row in LDS
    constexpr int KS = D / 32;      // k-steps of the QK product
    constexpr int DT = D / 16;      // 16-dim tiles of O^T
    __shared__ __align__(16) _Float16 sK[BKV * LDK];
    __shared__ __align__(16) _Float16 sVT[D * LDV];
    __shared__ int s_vote[2][WQ];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int hk = blockIdx.y;
    const int qv = blockIdx.x * (16 * WQ) + wave * 16 + j;  // this lane's query vector
    const bool qok = qv < NQ;
    const int64_t h = (int64_t)hk * G + (qok ? qv % G : 0);
    const int64_t qi = qok ? qv / G : 0;             // its query row (mask row, output row)

    // Q^T operand: dims 32 ks + 8 g .. +7 of query qv, hi and lo fp16 parts
    half8_t qh[KS], ql[KS];
    {
        const float* qp = reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(a.q) + qi * a.qnb1 +
                                                         h * a.qnb2);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = qok ? qp[32 * ks + 8 * g + e] : 0.0f;
                const _Float16 hi = (_Float16)x;
                qh[ks][e] = hi;
                ql[ks][e] = q_f16 ? (_Float16)0.0f : (_Float16)(x - (float)hi);
            }
    }
    float4_t o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;

    // K/V rows of this kv head as raw buffers over [0, n_kv): rows past n_kv read 0
    auto rsrc = [&](const void* p, int64_t nb2, int64_t nb1) {
        const uint64_t base = reinterpret_cast<uint64_t>(p) + (uint64_t)(hk * nb2);
        const int64_t bytes = a.n_kv * nb1;
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
        const uint32_t n = (uint32_t)(bytes > 0x7fffffff ? 0x7fffffff : bytes);
        return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                                 (int)__builtin_amdgcn_readfirstlane(n), 0x00020000);
    };
    const __amdgpu_buffer_rsrc_t krs = rsrc(a.k, a.knb2, a.knb1), vrs = rsrc(a.v, a.vnb2, a.vnb1);
    // staging: the block's 64 rows x D halves of K and of V in 16-byte pieces
    constexpr int PPR = D / 8;                 // pieces per row
    constexpr int NPC = BKV * PPR / (64 * WQ);  // pieces per thread per matrix (2 to 8)
    // thread -> piece column pc of NPC consecutive keys (each wave instruction reads
    // 4 or 8 whole rows), so V is transposed with one NPC-key write per dim
    const int ppc = tid % PPR, pr0 = NPC * (tid / PPR);
    u32x4 kreg[NPC], vreg[NPC];
    auto fetch = [&](int64_t c0) {
#pragma unroll
        for (int u = 0; u < NPC; ++u) {
            const int64_t row = c0 + pr0 + u;
            const uint32_t ko = row < a.n_kv ? (uint32_t)(row * a.knb1 + ppc * 16) : 0x80000000u;
            const uint32_t vo = row < a.n_kv ? (uint32_t)(row * a.vnb1 + ppc * 16) : 0x80000000u;
            kreg[u] = __builtin_amdgcn_raw_buffer_load_b128(krs, (int)ko, 0, 0);
            vreg[u] = __builtin_amdgcn_raw_buffer_load_b128(vrs, (int)vo, 0, 0);
        }
    };
    auto park = [&]() {
#pragma unroll
        for (int u = 0; u < NPC; ++u) *reinterpret_cast<u32x4*>(&sK[(pr0 + u) * LDK + ppc * 8]) = kreg[u];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint32_t hv[NPC];
#pragma unroll
            for (int u = 0; u < NPC; ++u) hv[u] = (vreg[u][e >> 1] >> (16 * (e & 1))) & 0xffffu;
            _Float16* dst = &sVT[(ppc * 8 + e) * LDV + pr0];
            if constexpr (NPC == 8) {
                *reinterpret_cast<uint4*>(dst) = make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16),
                                                            hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16));
            } else if constexpr (NPC == 4) {
                *reinterpret_cast<uint2*>(dst) = make_uint2(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16));
            } else {
                *reinterpret_cast<uint32_t*>(dst) = hv[0] | (hv[1] << 16);
            }
        }
    };

    const int nblk = (int)((a.n_kv + BKV - 1) / BKV);
    // Mask values of this lane's keys (16 t + 4 g + r) of a block: one 8-byte raw buffer
    // load per t, issued with the block's K/V prefetch (rows past S and missing masks
    // read 0 without a fetch; keys past n_kv and lanes without a query become -inf when
    // unpacked). With n_kv % 4 == 0 every 4-key group of a row lies inside the row;
    // other shapes, and row strides that are not a multiple of 8 bytes, take 2-byte loads.
    const bool m8 = a.mask && a.mnb1 % 8 == 0 && a.n_kv % 4 == 0 && (reinterpret_cast<uintptr_t>(a.mask) & 7) == 0;
    const __amdgpu_buffer_rsrc_t mrs = [&] {
        const uint64_t base = reinterpret_cast<uint64_t>(a.mask);
        const int64_t bytes = m8 ? a.S * a.mnb1 : 0;
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
        const uint32_t n = (uint32_t)(bytes > 0x7fffffff ? 0x7fffffff : bytes);
        return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                                 (int)__builtin_amdgcn_readfirstlane(n), 0x00020000);
    }();
    const uint8_t* mrow = a.mask && qok ? reinterpret_cast<const uint8_t*>(a.mask) + qi * a.mnb1 : nullptr;
    auto load_mask = [&](int64_t c0, uint32_t (&mw)[4][2]) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int64_t key = c0 + 16 * t + 4 * g;
            if (m8) {
                const uint32_t off = qok && key < a.n_kv ? (uint32_t)(qi * a.mnb1 + key * 2) : 0x80000000u;
                const auto v = __builtin_amdgcn_raw_buffer_load_b64(mrs, (int)off, 0, 0);
                mw[t][0] = v[0];
                mw[t][1] = v[1];
            } else {
                uint16_t h[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) h[r] = mrow && key + r < a.n_kv ? reinterpret_cast<const uint16_t*>(mrow)[key + r] : 0;
                mw[t][0] = h[0] | ((uint32_t)h[1] << 16);
                mw[t][1] = h[2] | ((uint32_t)h[3] << 16);
            }
        }
    };
    auto mask_val = [&](const uint32_t (&mw)[4][2], int64_t c0, int t, int r) -> float {
        const int64_t key = c0 + 16 * t + 4 * g + r;
        if (key >= a.n_kv || !qok) return -INFINITY;
        return h2f((uint16_t)(mw[t][r >> 1] >> (16 * (r & 1))));
    };
    // A block is skipped when every mask value the tile sees in it is -32768 or below
    // (the executor's masked value) and every query of the tile already holds a
    // running max from an unmasked key: exp(s - 32768 - m) is exactly 0 in fp32 then,
    // so the result is unchanged. (Causal prefill skips the blocks past the diagonal.)
    auto needed = [&](const uint32_t (&mw)[4][2], int64_t c0) -> int {
        bool any = qok && !(m > -16384.0f);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) any = any || mask_val(mw, c0, t, r) > -32768.0f;
        return any ? 1 : 0;
    };
    uint32_t mk[4][2], mkn[4][2];
    fetch(0);
    load_mask(0, mkn);
    for (int bi = 0; bi < nblk; ++bi) {
        const int64_t c0 = (int64_t)bi * BKV;
#pragma unroll
        for (int t = 0; t < 4; ++t) mk[t][0] = mkn[t][0], mk[t][1] = mkn[t][1];
        const int need = needed(mk, c0);
        // barrier: the previous block's LDS is fully read; and the skip decision (wave
        // votes in a slot per block parity: the next write to a slot follows a barrier
        // every wave passes only after reading it)
        // (the vote is taken by every lane before the branch: inside it, only lane 0 would
        // vote, and the block would be skipped when lane 0 alone does not need it)
        const int wneed = __any(need) ? 1 : 0;
        if (lane == 0) s_vote[bi & 1][wave] = wneed;
        __syncthreads();
        int vote = 0;
#pragma unroll
        for (int w = 0; w < WQ; ++w) vote |= s_vote[bi & 1][w];
        const bool run = vote != 0;
        if (run) {
            park();
            __syncthreads();
        }
        if (bi + 1 < nblk) {
            fetch(c0 + BKV);
            load_mask(c0 + BKV, mkn);
        }
        if (run) {
            // S^T tiles: keys 16 t .. 16 t + 15 x this wave's 16 queries
            float4_t st[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const half8_t kf = *reinterpret_cast<const half8_t*>(&sK[(16 * t + j) * LDK + 32 * ks + 8 * g]);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[ks], c, 0, 0, 0);
                    if (!q_f16) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[ks], c, 0, 0, 0);
                }
                st[t] = c;
            }
            // online softmax for query j: this lane's 16 keys, then lanes j + 16 g'
            float bmax = -INFINITY;
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float mv = mask_val(mk, c0, t, r);
                    const float sv = mv == -INFINITY ? -INFINITY : st[t][r] * a.scale + mv;
                    st[t][r] = sv;
                    bmax = fmaxf(bmax, sv);
                }
            {
                const Pair p16 = xchg_16(bmax);
                bmax = fmaxf(p16.a, p16.b);
                const Pair p32 = xchg_32(bmax);
                bmax = fmaxf(p32.a, p32.b);
            }
            const float mn = fmaxf(m, bmax);
            const float al = mn == -INFINITY ? 1.0f : __expf(m - mn);  // m = -inf: nothing accumulated yet
            // P^T operands: keys (32 kk + 4 g .. +3, 32 kk + 16 + 4 g .. +3), p = p_hi + p_lo in fp16
            half8_t pb[2], pl[2];
            float psum = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float pv = mn == -INFINITY ? 0.0f : __expf(st[t][r] - mn);
                    const _Float16 ph = (_Float16)pv;
                    psum += pv;
                    pb[t >> 1][4 * (t & 1) + r] = ph;
                    pl[t >> 1][4 * (t & 1) + r] = (_Float16)(pv - (float)ph);
                }
            {
                const Pair p16 = xchg_16(psum);
                psum = p16.a + p16.b;
                const Pair p32 = xchg_32(psum);
                psum = p32.a + p32.b;
            }
            l = l * al + psum;
            m = mn;
            // O^T (dims x queries) += V^T . P^T; V^T operand in the key order of pb
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                float4_t c = o[dt] * al;
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const _Float16* vr = &sVT[(16 * dt + j) * LDV + 32 * kk + 4 * g];
                    half8_t vf;
                    __builtin_memcpy(&vf, vr, 8);
                    __builtin_memcpy(reinterpret_cast<_Float16*>(&vf) + 4, vr + 16, 8);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pb[kk], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl[kk], c, 0, 0, 0);
                }
                o[dt] = c;
            }
        }
    }
    if (!qok) return;
    const float inv = l == 0.0f ? 0.0f : 1.0f / l;
    float* op = a.dst + (qi * a.Hq + h) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) op[16 * dt + 4 * g + r] = o[dt][r] * inv;
}

// Paged batched decode attention on the matrix cores for groups of 2..16 query heads
// per kv head (v_mfma_f32_16x16x32_f16, operand layouts as in k_attn_mma). A workgroup
// owns (split of 128 rows, kv head, sequence); wave w takes the split's keys 32 w .. +31:
//   S^T (16 keys x 16 queries, two tiles) = K . Q^T with K read straight into the MFMA
//   operand (16 bytes of one key row per lane) and Q rounded to fp16 (the decode path's
//   rounding); s = S * scale, keys at or past the sequence's length weigh 0;
//   O^T += V^T . P^T with P = p_hi + p_lo (fp32-level weights) and V transposed into the
//   wave's LDS slice (one packed write of 8 or 4 keys per dim).
// The 4 waves' (m, l, O) merge in LDS into the split's partial, which k_attn_merge
// combines across splits. Rows past a sequence's length (and missing pages) are never
// read: their loads use out-of-range offsets.
//
// The launch is a 1-D grid over a work list of (sequence, kv head, split) items that every
// wave rebuilds from the sequence lengths: workgroup i takes item i, so the splits that
// hold rows come first in dispatch order and the workgroups past the list's end (the
// grid is sized for max_len) exit last. (A (split, kv head, sequence) grid left resident
// slots to the empty splits of short sequences and ran working ones in a second round
// behind them: 2 x the time at 16 sequences of 2048 rows under max_len 4096.)
// Item i is kv head i % Hkv of split number i / Hkv in the list of every sequence's
// min(cdiv(len, 128), n_split) splits in sequence order (slen: that sequence's length);
// false past the list's end.
__device__ __forceinline__ bool paged_item(const PagedKv& pg, int n_split, int Hkv, int64_t i, int& seq, int& hk,
                                           int& split, int& slen, int64_t& n_items) {
    const int lane = threadIdx.x & 63;
    const int64_t c = i / Hkv;
    hk = (int)(i - c * Hkv);
    int64_t base = 0;  // splits of the sequences before this chunk of 64
    for (int b0 = 0; b0 < pg.B; b0 += 64) {
        const int b = b0 + lane;
        const int len = b < pg.B ? pg.len[b] : 0;
        const int n = len > 0 ? (int)min<int64_t>(cdiv(len, 128), n_split) : 0;
        int x = n;  // inclusive prefix sum over the chunk's lanes
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        const int tot = __shfl(x, 63, 64);
        if (c < base + tot) {
            // the sequences whose prefix ends at or before c precede the item's sequence
            const int k = __popcll(__ballot(base + x <= c));
            seq = b0 + k;
            split = (int)(c - base - __shfl(x - n, k, 64));
            slen = __shfl(len, k, 64);
            return true;
        }
        base += tot;
    }
    n_items = base * Hkv;
    return false;
}

// fuse (contiguous route only): 0 the merge runs in k_attn_merge, else 1 + the stream's
// counter set: the last workgroup of each kv head merges (G * D <= 256, n_split <=
// FUSE_MAX_SPLIT), as in k_attn_dec
template <int D>
__global__ __launch_bounds__(256) void k_attn_dec_mma(AttnArgs a, int G, int n_split, float* __restrict__ part,
                                                      PagedKv pg, int q16, int fuse = 0) {
    constexpr int KS = D / 32;         // k-steps of the QK product
    constexpr int DT = D / 16;         // 16-dim tiles of O^T
    constexpr int KW = 32;             // keys per wave
    constexpr int LDV = KW + 8;        // halves per V^T row
    constexpr int PPR = D / 8;         // 16-byte pieces per V row
    constexpr int KPL = KW * PPR / 64; // V keys per lane (8 or 4)
    constexpr int SV = D * LDV;        // halves of one wave's V^T slice
    __shared__ __align__(16) _Float16 sVT[4 * SV];
    __shared__ float sM[4][16], sL[4][16];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int Hkv = (int)a.Hkv;
    int seq_, hk_, split_, len_;
    if (pg.len) {
        int64_t n_items = 0;
        if (!paged_item(pg, n_split, Hkv, blockIdx.x, seq_, hk_, split_, len_, n_items)) {  // past the list
            // with one split the outputs are written here, not by the merge: the first
            // workgroup past the list (there is one per kv head of each sequence without
            // rows) writes zeros for those sequences, as the merge would
            if (n_split == 1 && (int64_t)blockIdx.x == n_items) {
                const int64_t per = a.Hq * D;
                for (int64_t idx = tid; idx < (int64_t)pg.B * per; idx += 256)
                    if (pg.len[idx / per] <= 0) a.dst[idx] = 0.0f;
            }
            return;
        }
    } else {  // one contiguous sequence of a.n_kv rows (no table: page i is rows 128 i ..)
        seq_ = 0;
        hk_ = (int)(blockIdx.x % (unsigned)Hkv);
        split_ = (int)(blockIdx.x / (unsigned)Hkv);
        len_ = (int)a.n_kv;
        if (split_ >= n_split) return;
    }
    const int seq = __builtin_amdgcn_readfirstlane(seq_), hk = __builtin_amdgcn_readfirstlane(hk_),
              split = __builtin_amdgcn_readfirstlane(split_);
    const int64_t r_begin = (int64_t)split * 128;
    const int64_t len = __builtin_amdgcn_readfirstlane(len_);
    const int64_t pi = r_begin >> pg.log2p;
    const int page = (r_begin < len && pi < pg.tstride) ? (pg.table ? pg.table[seq * pg.tstride + pi] : (int)pi) : -1;
    const int64_t r_len = page < 0 ? 0 : len;  // logical rows below r_len are read
    const int64_t prow0 = ((int64_t)(page < 0 ? 0 : page) << pg.log2p) + (r_begin & ((1 << pg.log2p) - 1));
    const int64_t kb0 = r_begin + wave * KW;   // this wave's first key (logical row)

    auto rsrc = [&](const void* p, int64_t nb2, int64_t nb1) {
        const uint64_t base = reinterpret_cast<uint64_t>(p) + (uint64_t)(hk * nb2);
        const int64_t bytes = a.n_kv * nb1;
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
        const uint32_t n = (uint32_t)(bytes > 0x7fffffff ? 0x7fffffff : bytes);
        return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                                 (int)__builtin_amdgcn_readfirstlane(n), 0x00020000);
    };
    const __amdgpu_buffer_rsrc_t krs = rsrc(a.k, a.knb2, a.knb1), vrs = rsrc(a.v, a.vnb2, a.vnb1);

    // K operands of both key tiles and this lane's V pieces, all requested at once
    u32x4 kw[2][KS];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int64_t r = kb0 + 16 * t + j;
        const bool in = r < r_len;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const uint32_t off = in ? (uint32_t)((prow0 + r - r_begin) * a.knb1 + (32 * ks + 8 * g) * 2) : 0x80000000u;
            kw[t][ks] = __builtin_amdgcn_raw_buffer_load_b128(krs, (int)off, 0, 0);
        }
    }
    const int pc = lane % PPR, kg = lane / PPR;
    u32x4 vreg[KPL];
#pragma unroll
    for (int u = 0; u < KPL; ++u) {
        const int64_t r = kb0 + kg * KPL + u;
        const uint32_t off = r < r_len ? (uint32_t)((prow0 + r - r_begin) * a.vnb1 + pc * 16) : 0x80000000u;
        vreg[u] = __builtin_amdgcn_raw_buffer_load_b128(vrs, (int)off, 0, 0);
    }

    // the KQ mask of a contiguous decode (one query row, 8-byte aligned): this lane's keys
    // 16 t + 4 g .. + 3 in one 8-byte load per t (keys past n_kv read 0 and are not used)
    u32x2 mk[2] = {{0u, 0u}, {0u, 0u}};
    if (a.mask) {
        const uint64_t mb = reinterpret_cast<uint64_t>(a.mask);
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)mb);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(mb >> 32));
        const __amdgpu_buffer_rsrc_t mrs = __builtin_amdgcn_make_buffer_rsrc(
            reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
            (int)__builtin_amdgcn_readfirstlane((uint32_t)(a.n_kv * 2)), 0x00020000);
#pragma unroll
        for (int t = 0; t < 2; ++t)
            mk[t] = __builtin_amdgcn_raw_buffer_load_b64(mrs, (int)((kb0 + 16 * t + 4 * g) * 2), 0, 0);
    }

    // Q^T operand: query j (lanes past G hold zeros), dims 32 ks + 8 g .. +7, fp16
    const bool qok = j < G;
    half8_t qh[KS];
    {
        const int64_t h = (int64_t)hk * G + (qok ? j : 0);
        const float* qp = reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(a.q) + seq * a.qnb1 +
                                                         h * a.qnb2);
        if (q16) {  // 16-byte aligned q rows: two 16-byte loads per 8 dims
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const float4 x0 = *reinterpret_cast<const float4*>(qp + 32 * ks + 8 * g);
                const float4 x1 = *reinterpret_cast<const float4*>(qp + 32 * ks + 8 * g + 4);
                const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) qh[ks][e] = (_Float16)(qok ? xv[e] : 0.0f);
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) qh[ks][e] = (_Float16)(qok ? qp[32 * ks + 8 * g + e] : 0.0f);
        }
    }

    // V^T into this wave's slice: dim pc * 8 + e, keys kg * KPL .. + KPL - 1 in one write
    _Float16* vt = sVT + wave * SV;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        uint32_t hv[KPL];
#pragma unroll
        for (int u = 0; u < KPL; ++u) hv[u] = (vreg[u][e >> 1] >> (16 * (e & 1))) & 0xffffu;
        _Float16* dst = vt + (pc * 8 + e) * LDV + kg * KPL;
        if constexpr (KPL == 8) {
            *reinterpret_cast<uint4*>(dst) =
                make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16));
        } else {
            *reinterpret_cast<uint2*>(dst) = make_uint2(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16));
        }
    }

    // S^T tiles: keys 16 t + 4 g + r of this wave x query j
    float sv[2][4];
    float bmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        float4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            half8_t kf;
            __builtin_memcpy(&kf, &kw[t][ks], 16);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[ks], c, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool ok = qok && kb0 + 16 * t + 4 * g + r < r_len;
            if (a.mask) {  // s = scale * q.k + mask, as the prefill kernel
                const float mv = h2f((uint16_t)(mk[t][r >> 1] >> (16 * (r & 1))));
                sv[t][r] = ok && mv != -INFINITY ? c[r] * a.scale + mv : -INFINITY;
            } else {
                sv[t][r] = ok ? c[r] * a.scale : -INFINITY;
            }
            bmax = fmaxf(bmax, sv[t][r]);
        }
    }
    {
        const Pair p16 = xchg_16(bmax);
        bmax = fmaxf(p16.a, p16.b);
        const Pair p32 = xchg_32(bmax);
        bmax = fmaxf(p32.a, p32.b);
    }
    const float m = bmax;
    // P^T operand (keys 4 g .. +3, 16 + 4 g .. +3), p = p_hi + p_lo in fp16
    half8_t pb, pl;
    float psum = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float pv = m == -INFINITY ? 0.0f : __expf(sv[t][r] - m);
            const _Float16 ph = (_Float16)pv;
            psum += pv;
            pb[4 * t + r] = ph;
            pl[4 * t + r] = (_Float16)(pv - (float)ph);
        }
    {
        const Pair p16 = xchg_16(psum);
        psum = p16.a + p16.b;
        const Pair p32 = xchg_32(psum);
        psum = p32.a + p32.b;
    }
    wave_lds_sync();  // the wave's V^T slice is written
    float4_t o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
        const _Float16* vr = vt + (16 * dt + j) * LDV + 4 * g;
        half8_t vf;
        __builtin_memcpy(&vf, vr, 8);
        __builtin_memcpy(reinterpret_cast<_Float16*>(&vf) + 4, vr + 16, 8);
        float4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pb, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl, c, 0, 0, 0);
        o[dt] = c;
    }

    // merge the 4 waves (the V^T slices are reused as sO[wave][dim][query])
    __syncthreads();
    float* sO = reinterpret_cast<float*>(sVT);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sO[(wave * D + 16 * dt + 4 * g + r) * 16 + j] = o[dt][r];
    if (g == 0) sM[wave][j] = m, sL[wave][j] = psum;
    __syncthreads();
    for (int idx = tid; idx < G * D; idx += 256) {
        const int u = idx / D, d = idx % D;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) mx = fmaxf(mx, sM[w][u]);
        float L = 0.0f, acc = 0.0f;
        if (mx != -INFINITY) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float f = sM[w][u] == -INFINITY ? 0.0f : __expf(sM[w][u] - mx);
                L += sL[w][u] * f;
                acc += sO[(w * D + d) * 16 + u] * f;
            }
        }
        const int64_t h = (int64_t)hk * G + u;
        if (n_split == 1) {
            a.dst[(seq * a.Hq + h) * D + d] = L == 0.0f ? 0.0f : acc / L;
        } else {
            float* pp = part + (((int64_t)split * Hkv + hk) * pg.B * G + (int64_t)seq * G + u) * (D + 2);
            if (fuse) {
                st_ag(pp + 2 + d, acc);
                if (d == 0) st_ag(pp, mx), st_ag(pp + 1, L);
            } else {
                pp[2 + d] = acc;
                if (d == 0) pp[0] = mx, pp[1] = L;
            }
        }
    }
    if (!fuse || n_split == 1) return;
    if (!arrive_last(&g_attn_arrive[(fuse - 1) * ARRIVE_N + hk], n_split)) return;
    const int u = tid / D, d = tid % D;
    if (u >= G) return;
    const float mo = merge_splits_ag(part + ((int64_t)hk * G + u) * (D + 2), (int64_t)Hkv * G * (D + 2), n_split, d);
    a.dst[((int64_t)hk * G + u) * D + d] = mo;
}

// the matrix-core prefill kernel: no ALiBi / softcap, 16-byte aligned K/V rows,
// buffer offsets within 2 GiB
bool mma_ok(const AttnArgs& a) {
    if (a.max_bias != 0.0f || a.softcap != 0.0f || (a.D != 64 && a.D != 128)) return false;
    if (a.knb1 % 16 || a.vnb1 % 16) return false;
    return a.n_kv * a.knb1 < 0x7fff0000LL && a.n_kv * a.vnb1 < 0x7fff0000LL;
}

template <int D>
__global__ __launch_bounds__(256) void k_attn(AttnArgs a, int G, int NQ, int cps, int n_chunks, int n_split,
                                              float m0, float m1, uint32_t n_head_log2, int q_f16,
                                              float* __restrict__ part) {
    constexpr int LDV = D + 8;  // halves per LDS row
    __shared__ __align__(16) float sQ[QT][D];
    __shared__ __align__(16) uint16_t sK[CH * LDV];
    __shared__ __align__(16) uint16_t sV[CH * LDV];
    __shared__ float sS[QT][CH];
    __shared__ float sM[QT], sL[QT], sA[QT];

    const int tid = threadIdx.x;
    const int split = blockIdx.x;
    const int hk = blockIdx.y;
    const int qt = blockIdx.z;
    const int Hkv = (int)a.Hkv;

    // ---- query tile -> LDS
    for (int idx = tid; idx < QT * D; idx += 256) {
        const int qq = idx / D, d = idx % D;
        const int qv = qt * QT + qq;
        float val = 0.0f;
        if (qv < NQ && d < a.D) {  // head dims padded to the template's D: 0
            const int64_t h = (int64_t)hk * G + qv % G;
            const int64_t i = qv / G;
            val = *reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(a.q) + i * a.qnb1 +
                                                  h * a.qnb2 + (int64_t)d * 4);
            if (q_f16) val = (float)(_Float16)val;
        }
        sQ[qq][d] = val;
    }
    if (tid < QT) {
        sM[tid] = -INFINITY;
        sL[tid] = 0.0f;
    }

    // phase-3 mapping: lane owns 2 dims of QPG query vectors
    constexpr int TPQ = D / 2;          // threads per query group
    constexpr int NQG = 256 / TPQ;      // query groups (4 or 8)
    constexpr int QPG = QT / NQG;       // queries per group (4 or 2)
    const int od = (tid % TPQ) * 2;
    const int oqg = tid / TPQ;
    float o[QPG][2];
#pragma unroll
    for (int u = 0; u < QPG; ++u) o[u][0] = o[u][1] = 0.0f;

    // phase-1 mapping: lane owns one kv row and 4 query vectors
    const int sr = tid & 63;
    const int sqg = tid >> 6;

    const int c_begin = split * cps;
    const int c_end = min(n_chunks, c_begin + cps);
    const uint8_t* kbase = reinterpret_cast<const uint8_t*>(a.k) + (int64_t)hk * a.knb2;
    const uint8_t* vbase = reinterpret_cast<const uint8_t*>(a.v) + (int64_t)hk * a.vnb2;

    for (int c = c_begin; c < c_end; ++c) {
        const int64_t c0 = (int64_t)c * CH;
        const int rows = (int)min<int64_t>(CH, a.n_kv - c0);
        __syncthreads();
        // ---- K/V chunk -> LDS (16-byte pieces)
        constexpr int PPR = D / 8;  // pieces per row
        for (int idx = tid; idx < CH * PPR; idx += 256) {
            const int r = idx / PPR, pc = idx % PPR;
            uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
            if (r < rows && pc * 8 < a.D) {
                kv = *reinterpret_cast<const uint4*>(kbase + (c0 + r) * a.knb1 + pc * 16);
                vv = *reinterpret_cast<const uint4*>(vbase + (c0 + r) * a.vnb1 + pc * 16);
            }
            *reinterpret_cast<uint4*>(&sK[r * LDV + pc * 8]) = kv;
            *reinterpret_cast<uint4*>(&sV[r * LDV + pc * 8]) = vv;
        }
        __syncthreads();
        // ---- scores
        {
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
            for (int d = 0; d < D; d += 8) {
                const uint4 kp = *reinterpret_cast<const uint4*>(&sK[sr * LDV + d]);
                float kf[8];
                const uint32_t kw[4] = {kp.x, kp.y, kp.z, kp.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    kf[2 * e] = h2f((uint16_t)(kw[e] & 0xffff));
                    kf[2 * e + 1] = h2f((uint16_t)(kw[e] >> 16));
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float4 qa = *reinterpret_cast<const float4*>(&sQ[sqg + 4 * u][d]);
                    const float4 qb = *reinterpret_cast<const float4*>(&sQ[sqg + 4 * u][d + 4]);
                    acc[u] += qa.x * kf[0] + qa.y * kf[1] + qa.z * kf[2] + qa.w * kf[3] + qb.x * kf[4] +
                              qb.y * kf[5] + qb.z * kf[6] + qb.w * kf[7];
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int qq = sqg + 4 * u;
                const int qv = qt * QT + qq;
                float s = -INFINITY;
                if (sr < rows && qv < NQ) {
                    s = acc[u] * a.scale;
                    if (a.softcap != 0.0f) s = a.softcap * tanhf(s);
                    if (a.mask) {
                        const int64_t h = (int64_t)hk * G + qv % G;
                        const int64_t i = qv / G;
                        float slope = 1.0f;
                        if (a.max_bias > 0.0f)
                            slope = h < n_head_log2 ? powf(m0, (float)(h + 1))
                                                    : powf(m1, (float)(2 * (h - n_head_log2) + 1));
                        const uint16_t mv = *reinterpret_cast<const uint16_t*>(
                            reinterpret_cast<const uint8_t*>(a.mask) + i * a.mnb1 + (c0 + sr) * 2);
                        const float mf = slope * h2f(mv);
                        s = mf == -INFINITY ? -INFINITY : s + mf;
                    }
                }
                sS[qq][sr] = s;
            }
        }
        __syncthreads();
        // ---- online softmax update (16 lanes per query vector)
        {
            const int qq = tid >> 4, sub = tid & 15;
            float sv[4];
            float mx = -INFINITY;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                sv[k] = sS[qq][sub + 16 * k];
                mx = fmaxf(mx, sv[k]);
            }
            mx = xor_max<16>(mx);
            const float mold = sM[qq];
            const float mnew = fmaxf(mold, mx);
            float ps = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float p = mnew == -INFINITY ? 0.0f : __expf(sv[k] - mnew);
                sS[qq][sub + 16 * k] = p;
                ps += p;
            }
            ps = xor_sum<16>(ps);
            if (sub == 0) {
                const float alpha = mnew == -INFINITY ? 1.0f : __expf(mold - mnew);
                sA[qq] = alpha;
                sM[qq] = mnew;
                sL[qq] = sL[qq] * alpha + ps;
            }
        }
        __syncthreads();
        // ---- O += P V
        {
#pragma unroll
            for (int u = 0; u < QPG; ++u) {
                const float al = sA[oqg * QPG + u];
                o[u][0] *= al;
                o[u][1] *= al;
            }
            for (int r = 0; r < rows; ++r) {
                const uint32_t vw = *reinterpret_cast<const uint32_t*>(&sV[r * LDV + od]);
                const float v0 = h2f((uint16_t)(vw & 0xffff)), v1 = h2f((uint16_t)(vw >> 16));
#pragma unroll
                for (int u = 0; u < QPG; ++u) {
                    const float p = sS[oqg * QPG + u][r];
                    o[u][0] += p * v0;
                    o[u][1] += p * v1;
                }
            }
        }
    }
    __syncthreads();

#pragma unroll
    for (int u = 0; u < QPG; ++u) {
        const int qq = oqg * QPG + u;
        const int qv = qt * QT + qq;
        if (qv >= NQ) continue;
        const int64_t h = (int64_t)hk * G + qv % G;
        const int64_t i = qv / G;
        if (n_split == 1) {
            const float L = sL[qq];
            const float inv = L == 0.0f ? 0.0f : 1.0f / L;
            if (od < a.D) {  // a.D % 8 == 0: both dims or neither
                float* op = a.dst + (i * a.Hq + h) * a.D + od;
                op[0] = o[u][0] * inv;
                op[1] = o[u][1] * inv;
            }
        } else {
            float* pp = part + (((int64_t)split * Hkv + hk) * NQ + qv) * (D + 2);
            pp[2 + od] = o[u][0];
            pp[2 + od + 1] = o[u][1];
            if (od == 0) {
                pp[0] = sM[qq];
                pp[1] = sL[qq];
            }
        }
    }
}

// Merge of split partials (ops.cpp:9060-9128): weights w_s = exp(m_s - max) are
// computed once in LDS, then each thread sums its dimension over the splits with
// independent loads.
// With `len` (paged batches), query vector qv belongs to sequence qv / G and only its
// first cdiv(len, rps) splits hold partials (the splits past a sequence's length are not
// computed); without it every split does.
// With q8 (batched decode, NQ / G <= 16 sequences), the output rows are also written
// quantized for the output projection: row i (Hq * D values) in quant blocks of 32
// dims, each inside one half wave (the amax and block sum by xor shuffles), with
// quantize_row_q8_0's rule as quant8_block, into the int8 activation layout of
// act_prep_i8 (quants at (j * 16 + i) * 32, scale and block sum after all the quants).
template <int D>
__global__ __launch_bounds__(D) void k_attn_merge(const float* __restrict__ part, int n_split, int Hkv, int NQ,
                                                  int G, int64_t Hq, float* __restrict__ dst,
                                                  const int32_t* __restrict__ len = nullptr, int rps = 1,
                                                  uint8_t* __restrict__ q8 = nullptr, int Dr = D) {
    __shared__ float sW[MAX_SPLIT], sL[MAX_SPLIT];
    __shared__ float sRed[D / 64 > 0 ? D / 64 : 1];
    const int qv = blockIdx.x;
    const int hk = blockIdx.y;
    const int d = threadIdx.x;
    if (len) n_split = min(n_split, (int)cdiv(max(len[qv / G], 0), rps));
    const int64_t stride = (int64_t)Hkv * NQ * (D + 2);
    const float* base = part + ((int64_t)hk * NQ + qv) * (D + 2);
    float mx = -INFINITY;
    for (int s = d; s < n_split; s += D) {
        const float ms = base[s * stride], ls = base[s * stride + 1];
        const float mv = ls == 0.0f ? -INFINITY : ms;
        sW[s] = mv;
        sL[s] = ls;
        mx = fmaxf(mx, mv);
    }
    // up to MERGE_REG splits: every split's o is requested right behind the (m, l) loads,
    // before the max is known, so the partials arrive in one memory round trip. The loads
    // are unconditional (splits past n_split reread the last one) and the sums below skip
    // those splits by selects, in the same order as the loop.
    constexpr int MERGE_REG = 32;
    const bool in_reg = n_split <= MERGE_REG;
    float po[MERGE_REG];
    __builtin_amdgcn_sched_barrier(0);
    if (in_reg) {
        const int last = max(n_split - 1, 0);
#pragma unroll
        for (int s = 0; s < MERGE_REG; ++s) po[s] = base[min(s, last) * stride + 2 + d];
    }
    __builtin_amdgcn_sched_barrier(0);
    mx = xor_max<64>(mx);
    if ((d & 63) == 0) sRed[d >> 6] = mx;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < D / 64; ++w) mx = fmaxf(mx, sRed[w]);
    __syncthreads();
    for (int s = d; s < n_split; s += D) sW[s] = sW[s] == -INFINITY ? 0.0f : __expf(sW[s] - mx);
    __syncthreads();
    float L = 0.0f, acc = 0.0f;
    if (in_reg) {
#pragma unroll
        for (int s = 0; s < MERGE_REG; ++s) {
            const bool on = s < n_split;  // entries past n_split are read, never used
            const float w = sW[s], ls = sL[s];
            const float L1 = L + ls * w, a1 = acc + po[s] * w;
            L = on ? L1 : L;
            acc = on ? a1 : acc;
        }
    } else {  // chunks of MERGE_REG splits, each chunk's loads at once, the same order
        const int last = n_split - 1;
        for (int s0 = 0; s0 < n_split; s0 += MERGE_REG) {
#pragma unroll
            for (int s = 0; s < MERGE_REG; ++s) po[s] = base[min(s0 + s, last) * stride + 2 + d];
#pragma unroll
            for (int s = 0; s < MERGE_REG; ++s) {
                const int k = s0 + s;
                const bool on = k < n_split;  // entries past n_split are read, never used
                const int kk = min(k, MAX_SPLIT - 1);
                const float w = sW[kk], ls = sL[kk];
                const float L1 = L + ls * w, a1 = acc + po[s] * w;
                L = on ? L1 : L;
                acc = on ? a1 : acc;
            }
        }
    }
    const int64_t h = (int64_t)hk * G + qv % G;
    const int64_t i = qv / G;
    const float o = L == 0.0f ? 0.0f : acc / L;
    if (d < Dr) dst[(i * Hq + h) * Dr + d] = o;  // Dr: the head dim, D its padded width
    if (!q8) return;
    float amax = fabsf(o);
#pragma unroll
    for (int k = 1; k < 32; k <<= 1) amax = fmaxf(amax, __shfl_xor(amax, k, 64));
    const float dq = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    int q = (int)__builtin_rintf(o * id);
    q = q > 127 ? 127 : (q < -128 ? -128 : q);
    int qs = q;
#pragma unroll
    for (int k = 1; k < 32; k <<= 1) qs += __shfl_xor(qs, k, 64);
    const int64_t nbq = Hq * Dr / 32;                  // quant blocks of a row
    const int64_t e = ((h * Dr + d) / 32) * 16 + i;  // (block, row)
    q8[e * 32 + (d & 31)] = (uint8_t)(q & 0xff);
    if ((d & 31) == 0) {
        *reinterpret_cast<float*>(q8 + nbq * 512 + e * 4) = h2f(f2h(dq));
        *reinterpret_cast<int*>(q8 + nbq * 576 + e * 4) = qs;
    }
}

__global__ void k_attn_reset_counters() {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < ARRIVE_SETS * ARRIVE_N) g_attn_arrive[i] = 0u;
}

// the split merge (len, rps: the paged launches' per-sequence split counts; q8: the
// quantized output rows); D: the head dim, padded to 64, 128 or 256 for the partials
int launch_merge(int64_t D, const float* part, int ns, int Hkv, int NQ, int G, int64_t Hq, float* dst,
                 const int32_t* len, int rps, hipStream_t s, uint8_t* q8 = nullptr) {
    const dim3 g2((unsigned)NQ, (unsigned)Hkv);
    const int Dr = (int)D;
    if (D > 128)
        hipLaunchKernelGGL(k_attn_merge<256>, g2, dim3(256), 0, s, part, ns, Hkv, NQ, G, Hq, dst, len, rps, q8, Dr);
    else if (D > 64)
        hipLaunchKernelGGL(k_attn_merge<128>, g2, dim3(128), 0, s, part, ns, Hkv, NQ, G, Hq, dst, len, rps, q8, Dr);
    else
        hipLaunchKernelGGL(k_attn_merge<64>, g2, dim3(64), 0, s, part, ns, Hkv, NQ, G, Hq, dst, len, rps, q8, Dr);
    return check_hip(hipGetLastError(), "attention merge launch");
}

}  // namespace

int attn_reset_counters(hipStream_t s) {
    hipLaunchKernelGGL(k_attn_reset_counters, dim3(ARRIVE_SETS * ARRIVE_N / 256), dim3(256), 0, s);
    return check_hip(hipGetLastError(), "attn_reset_counters launch");
}

// the shapes a contiguous decode may run on k_attn_dec_mma (the strides and alignments
// decide at the call, contig_mma_ok)
bool contig_mma_shape(int64_t D, int64_t S, int64_t Hq, int64_t Hkv) {
    if (S != 1 || Hkv <= 0 || Hq % Hkv) return false;
    const int64_t G = Hq / Hkv;
    return (D == 64 || D == 128) && G > 1 && G <= 16;
}

// one query row of 2..16 query heads per kv head on the matrix cores (the paged kernel with
// 128-row pages that are the cache's own rows): head dim 64 or 128, no ALiBi or softcap,
// 16-byte K/V rows, an 8-byte aligned mask row, buffer offsets within 2 GiB
bool contig_mma_ok(const AttnArgs& a) {
    if (!contig_mma_shape(a.D, a.S, a.Hq, a.Hkv) || a.max_bias != 0.0f || a.softcap != 0.0f) return false;
    if (a.knb1 % 16 || a.vnb1 % 16 || (a.mask && (reinterpret_cast<uintptr_t>(a.mask) & 7))) return false;
    // the mask is read 4 keys per 8-byte load, bounded at n_kv keys: a multiple of 4 keeps
    // every key's load inside the bound (other lengths take k_attn_dec)
    if (a.mask && a.n_kv % 4) return false;
    if (a.n_kv < 1 || a.n_kv * a.knb1 >= 0x7fff0000LL || a.n_kv * a.vnb1 >= 0x7fff0000LL) return false;
    return cdiv(a.n_kv, 128) <= MAX_SPLIT;
}

size_t attn_workspace_bytes(int64_t D, int64_t S, int64_t Hq, int64_t Hkv, int64_t n_kv) {
    if (Hkv <= 0 || Hq % Hkv) return 0;
    const Plan p = make_plan(D, S, Hq, Hkv, n_kv);
    size_t need = p.n_split <= 1 ? 0 : (size_t)p.n_split * Hkv * p.NQ * (attn_width(D) + 2) * sizeof(float);
    if (contig_mma_shape(D, S, Hq, Hkv) && n_kv > 128 && cdiv(n_kv, 128) <= MAX_SPLIT) {  // 128-row splits
        const size_t mma = (size_t)cdiv(n_kv, 128) * Hkv * (Hq / Hkv) * (D + 2) * sizeof(float);
        need = need > mma ? need : mma;
    }
    return need;
}

int attention_contig_mma(const AttnArgs& a, void* ws, size_t ws_bytes, hipStream_t s) {
    const int64_t G = a.Hq / a.Hkv, ns = cdiv(a.n_kv, 128);
    const size_t need = attn_workspace_bytes(a.D, a.S, a.Hq, a.Hkv, a.n_kv);
    if (ns > 1 && (ws == nullptr || ws_bytes < need))
        return fail(GQ_ERR_WORKSPACE, "flash_attn_ext: workspace too small (need " + std::to_string(need) + " bytes)");
    float* part = reinterpret_cast<float*>(ws);
    const PagedKv pg{nullptr, nullptr, ns, 7, 1};
    const int q16 = (reinterpret_cast<uintptr_t>(a.q) & 15) == 0 && a.qnb1 % 16 == 0 && a.qnb2 % 16 == 0;
    const dim3 g1((unsigned)(ns * a.Hkv));
    // the last workgroup of each kv head merges when one thread per (query head, dim) fits
    // the workgroup (SmolLM2: 3 x 64); larger groups keep the merge launch
    const int set = fuse_merge_ok(ns, G, a.D, a.Hkv) ? arrive_set(s) : -1;
    if (a.D == 128)
        hipLaunchKernelGGL(k_attn_dec_mma<128>, g1, dim3(256), 0, s, a, (int)G, (int)ns, part, pg, q16, set + 1);
    else
        hipLaunchKernelGGL(k_attn_dec_mma<64>, g1, dim3(256), 0, s, a, (int)G, (int)ns, part, pg, q16, set + 1);
    const int rc = check_hip(hipGetLastError(), "flash_attn_ext (mfma decode) launch");
    if (rc != GQ_OK || ns == 1 || set >= 0) return rc;
    return launch_merge(a.D, part, (int)ns, (int)a.Hkv, (int)G, (int)G, a.Hq, a.dst, nullptr, 1, s);
}

int attention(const AttnArgs& a, void* ws, size_t ws_bytes, hipStream_t s) {
    if (contig_mma_ok(a)) return attention_contig_mma(a, ws, ws_bytes, s);
    const Plan p = make_plan(a.D, a.S, a.Hq, a.Hkv, a.n_kv);
    if (p.n_split > MAX_SPLIT) return fail(GQ_ERR_INVALID, "flash_attn_ext: context too long for one launch");
    const size_t need = attn_workspace_bytes(a.D, a.S, a.Hq, a.Hkv, a.n_kv);
    if (need > 0 && (ws == nullptr || ws_bytes < need))
        return fail(GQ_ERR_WORKSPACE, "flash_attn_ext: workspace too small (need " + std::to_string(need) + " bytes)");
    const uint32_t n_head = (uint32_t)a.Hq;
    const uint32_t n_head_log2 = 1u << (uint32_t)floor(log2((double)n_head));
    const float m0 = powf(2.0f, -(a.max_bias) / n_head_log2);
    const float m1 = powf(2.0f, -(a.max_bias / 2.0f) / n_head_log2);
    AttnArgs b = a;
    if (b.softcap != 0.0f) b.scale /= b.softcap;
    const int q_f16 = a.S < 64 ? 1 : 0;
    const int q_al = (reinterpret_cast<uintptr_t>(a.q) & 15) == 0 && a.qnb1 % 16 == 0 && a.qnb2 % 16 == 0;
    float* part = reinterpret_cast<float*>(ws);
    const int64_t W = attn_width(a.D);
    const int set = p.dec && fuse_merge_ok(p.n_split, p.NQ, W, a.Hkv) ? arrive_set(s) : -1;
    const bool fused_merge = set >= 0;
    if (p.dec) {
        const dim3 gd((unsigned)p.n_split, (unsigned)a.Hkv);
        const int nq = (int)p.NQ, G = (int)p.G, ns = (int)p.n_split;
        const int fuse = set + 1;
#define GQ_DEC(DD, NN, UU)                                                                                       \
    hipLaunchKernelGGL((k_attn_dec<DD, NN, UU, false>), gd, dim3(256), 0, s, b, G, nq, p.rows_per_split, ns, m0, m1, \
                       n_head_log2, q_f16 | (q_al << 1), part, PagedKv{}, fuse)
#define GQ_DEC_U(DD, NN)                           \
    do {                                           \
        if (p.dec_u == 8) GQ_DEC(DD, NN, 8);       \
        else if (p.dec_u == 4) GQ_DEC(DD, NN, 4);  \
        else GQ_DEC(DD, NN, 2);                    \
    } while (0)
        if (W == 256) {
            if (nq == 1) GQ_DEC_U(256, 1);
            else if (nq == 2) GQ_DEC_U(256, 2);
            else if (nq <= 4) GQ_DEC_U(256, 4);
            else if (p.dec_u == 4) GQ_DEC(256, 8, 4);
            else GQ_DEC(256, 8, 2);
        } else if (W == 128) {
            if (nq == 1 && p.dec_u == 12) GQ_DEC(128, 1, 12);
            else if (nq == 1 && p.dec_u == 10) GQ_DEC(128, 1, 10);
            else if (nq == 1) GQ_DEC_U(128, 1);
            else if (nq == 2) GQ_DEC_U(128, 2);
            else if (nq <= 4) GQ_DEC_U(128, 4);
            else if (p.dec_u == 4) GQ_DEC(128, 8, 4);  // u <= 4 for more than 4 query vectors
            else GQ_DEC(128, 8, 2);
        } else {
            if (nq == 1) GQ_DEC_U(64, 1);
            else if (nq == 2) GQ_DEC_U(64, 2);
            else if (nq <= 4) GQ_DEC_U(64, 4);
            else if (p.dec_u == 4) GQ_DEC(64, 8, 4);
            else GQ_DEC(64, 8, 2);
        }
#undef GQ_DEC_U
#undef GQ_DEC
    } else if (mma_ok(a)) {
        // tiles of 32 query vectors where tiles of 64 leave more than half the CUs idle
        // (Qwen2.5-1.5B shape at 512 tokens, 12 / 2 heads: 96 -> 192 workgroups, 34.1 ->
        // 29.6 us; the 7B's 256 workgroups of 64 are faster than 512 of 32: 37.3 / 40.7 us)
        if (cdiv(p.NQ, 64) * a.Hkv < 128) {
            const dim3 gm((unsigned)cdiv(p.NQ, 32), (unsigned)a.Hkv);
            if (a.D == 128)
                hipLaunchKernelGGL((k_attn_mma<128, 2>), gm, dim3(128), 0, s, b, (int)p.G, (int)p.NQ, q_f16);
            else
                hipLaunchKernelGGL((k_attn_mma<64, 2>), gm, dim3(128), 0, s, b, (int)p.G, (int)p.NQ, q_f16);
            return check_hip(hipGetLastError(), "flash_attn_ext (mfma) launch");
        }
        const dim3 gm((unsigned)cdiv(p.NQ, 64), (unsigned)a.Hkv);
        if (a.D == 128)
            hipLaunchKernelGGL(k_attn_mma<128>, gm, dim3(256), 0, s, b, (int)p.G, (int)p.NQ, q_f16);
        else
            hipLaunchKernelGGL(k_attn_mma<64>, gm, dim3(256), 0, s, b, (int)p.G, (int)p.NQ, q_f16);
        return check_hip(hipGetLastError(), "flash_attn_ext (mfma) launch");
    } else {
    const dim3 grid((unsigned)p.n_split, (unsigned)a.Hkv, (unsigned)p.n_qt);
    if (W == 256)
        hipLaunchKernelGGL(k_attn<256>, grid, dim3(256), 0, s, b, (int)p.G, (int)p.NQ, (int)p.cps, (int)p.n_chunks,
                           (int)p.n_split, m0, m1, n_head_log2, q_f16, part);
    else if (W == 128)
        hipLaunchKernelGGL(k_attn<128>, grid, dim3(256), 0, s, b, (int)p.G, (int)p.NQ, (int)p.cps, (int)p.n_chunks,
                           (int)p.n_split, m0, m1, n_head_log2, q_f16, part);
    else
        hipLaunchKernelGGL(k_attn<64>, grid, dim3(256), 0, s, b, (int)p.G, (int)p.NQ, (int)p.cps, (int)p.n_chunks,
                           (int)p.n_split, m0, m1, n_head_log2, q_f16, part);
    }
    int rc = check_hip(hipGetLastError(), "flash_attn_ext launch");
    if (rc != GQ_OK || p.n_split == 1 || fused_merge) return rc;
    return launch_merge(a.D, part, (int)p.n_split, (int)a.Hkv, (int)p.NQ, (int)p.G, a.Hq, a.dst, nullptr, 1, s);
}

namespace {

struct PagedPlan {
    int u;  // rows per lane stream of k_attn_dec; -1: k_attn_dec_mma
    int64_t rps, n_split;
};

// groups of 2..16 query heads per kv head go to the matrix-core kernel (pages of a
// multiple of 128 rows); one query head per kv head stays on the VALU kernel
bool paged_mma(int64_t D, int64_t G, int64_t page) {
    return (D == 64 || D == 128) && G > 1 && G <= 16 && page % 128 == 0;
}

// the largest rows-per-lane-stream U (8, 4, 2; at most 4 for more than 4 query vectors)
// whose split (U x rows per iteration) divides the page and still gives >= 256 workgroups
PagedPlan paged_plan(int64_t D, int64_t B, int64_t G, int64_t Hkv, int64_t max_len, int64_t page) {
    const int64_t rows_it = 4 * (64 / (D / 8));
    PagedPlan p{0, 0, 0};
    if (paged_mma(D, G, page))  // matrix-core kernel: splits of 128 rows (u = 0 marks it)
        return PagedPlan{-1, 128, cdiv(max_len < 1 ? 1 : max_len, 128)};
    for (int u = G > 4 ? 4 : 8; u >= 2; u >>= 1) {  // a smaller U replaces a larger one: more workgroups
        const int64_t rps = u * rows_it;
        if (page % rps) continue;
        p = PagedPlan{u, rps, cdiv(max_len < 1 ? 1 : max_len, rps)};
        if (B * Hkv * p.n_split >= DEC_TARGET_WG / 2 && p.n_split <= MAX_SPLIT) break;
    }
    return p;
}

}  // namespace

bool attention_paged_q8_ok(int64_t D, int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len, int64_t page) {
    if (Hkv <= 0 || Hq % Hkv || B > GEMM_I8_MAX_M) return false;
    const PagedPlan p = paged_plan(D, B, Hq / Hkv, Hkv, max_len, page);
    return p.u < 0 && p.n_split > 1;
}

size_t attn_paged_workspace_bytes(int64_t D, int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len, int64_t page) {
    if (Hkv <= 0 || Hq % Hkv) return 0;
    const PagedPlan p = paged_plan(D, B, Hq / Hkv, Hkv, max_len, page);
    if (p.u == 0 || p.n_split <= 1) return 0;
    return (size_t)p.n_split * Hkv * B * (Hq / Hkv) * (D + 2) * sizeof(float);
}

int attention_paged(const AttnArgs& a, const PagedKv& pg, int64_t max_len, void* ws, size_t ws_bytes, hipStream_t s,
                    uint8_t* q8) {
    const int64_t G = a.Hq / a.Hkv, page = (int64_t)1 << pg.log2p;
    const PagedPlan p = paged_plan(a.D, pg.B, G, a.Hkv, max_len, page);
    if (p.u == 0) return fail(GQ_ERR_INVALID, "flash_attn_paged: page size must be a multiple of 64 rows (128 for D = 64)");
    if (p.n_split > MAX_SPLIT) return fail(GQ_ERR_INVALID, "flash_attn_paged: context too long for one launch");
    const size_t need = attn_paged_workspace_bytes(a.D, pg.B, a.Hq, a.Hkv, max_len, page);
    if (need > 0 && (ws == nullptr || ws_bytes < need))
        return fail(GQ_ERR_WORKSPACE, "flash_attn_paged: workspace too small (need " + std::to_string(need) + " bytes)");
    float* part = reinterpret_cast<float*>(ws);
    const dim3 gd((unsigned)p.n_split, (unsigned)a.Hkv, (unsigned)pg.B);
    const int nq = (int)G, ns = (int)p.n_split;
    if (p.u < 0) {
        const dim3 g1((unsigned)(p.n_split * a.Hkv * pg.B));  // one workgroup per possible item
        const int q16 = (reinterpret_cast<uintptr_t>(a.q) & 15) == 0 && a.qnb1 % 16 == 0 && a.qnb2 % 16 == 0;
        if (a.D == 128)
            hipLaunchKernelGGL(k_attn_dec_mma<128>, g1, dim3(256), 0, s, a, nq, ns, part, pg, q16);
        else
            hipLaunchKernelGGL(k_attn_dec_mma<64>, g1, dim3(256), 0, s, a, nq, ns, part, pg, q16);
        int rc = check_hip(hipGetLastError(), "flash_attn_paged (mfma) launch");
        if (rc != GQ_OK || p.n_split == 1) return rc;
        return launch_merge(a.D, part, ns, (int)a.Hkv, (int)(pg.B * G), (int)G, a.Hq, a.dst, pg.len, 128, s, q8);
    }
    const int set = fuse_merge_ok(p.n_split, G, a.D, a.Hkv * pg.B) ? arrive_set(s) : -1;
    const bool fused_merge = set >= 0;
    const int q_al = (reinterpret_cast<uintptr_t>(a.q) & 15) == 0 && a.qnb1 % 16 == 0 && a.qnb2 % 16 == 0;
    const int fuse = set + 1;
#define GQ_PDEC(DD, NN, UU)                                                                                        \
    hipLaunchKernelGGL((k_attn_dec<DD, NN, UU, true>), gd, dim3(256), 0, s, a, nq, nq, p.rps, ns, 1.0f, 1.0f, 1u, \
                       1 | (q_al << 1), part, pg, fuse)
#define GQ_PDEC_U(DD, NN)                          \
    do {                                           \
        if (p.u == 8) GQ_PDEC(DD, NN, 8);          \
        else if (p.u == 4) GQ_PDEC(DD, NN, 4);     \
        else GQ_PDEC(DD, NN, 2);                   \
    } while (0)
    if (a.D == 128) {
        if (nq == 1) GQ_PDEC_U(128, 1);
        else if (nq == 2) GQ_PDEC_U(128, 2);
        else if (nq <= 4) GQ_PDEC_U(128, 4);
        else if (p.u == 4) GQ_PDEC(128, 8, 4);
        else GQ_PDEC(128, 8, 2);
    } else {
        if (nq == 1) GQ_PDEC_U(64, 1);
        else if (nq == 2) GQ_PDEC_U(64, 2);
        else if (nq <= 4) GQ_PDEC_U(64, 4);
        else if (p.u == 4) GQ_PDEC(64, 8, 4);
        else GQ_PDEC(64, 8, 2);
    }
#undef GQ_PDEC_U
#undef GQ_PDEC
    int rc = check_hip(hipGetLastError(), "flash_attn_paged launch");
    if (rc != GQ_OK || p.n_split == 1 || fused_merge) return rc;
    return launch_merge(a.D, part, ns, (int)a.Hkv, (int)(pg.B * G), (int)G, a.Hq, a.dst, nullptr, 1, s);
}

// ---- allocation-free decode attention -------------------------------------
// gq_flash_attn_ext_noalloc takes its split partials from this file-scope device
// array instead of a caller workspace. Each device that loads the library holds its
// own copy (at its own address) until the process ends; in host code the name
// `scratch` is only a host-side stand-in, so kernels get the device address looked up
// once per device with hipGetSymbolAddress. Every partial a launch reads was written
// by the same launch, so nothing is cleared between calls; calls that overlap on one
// device race on it.
namespace {
static __device__ __align__(256) unsigned char scratch[ATTN_SCRATCH_BYTES];
constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[SCRATCH_MAX_DEVICES] = {};
}  // namespace

int attn_scratch_init(void** out) {
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) return fail(GQ_ERR_UNSUPPORTED, "attention scratch: device index too large");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(attention scratch)");
        if (rc) return rc;
        g_scratch_ptr[dev] = p;
    }
    if (out) *out = g_scratch_ptr[dev];
    return GQ_OK;
}

int attention_noalloc(const AttnArgs& a, hipStream_t s) {
    const size_t need = attn_workspace_bytes(a.D, a.S, a.Hq, a.Hkv, a.n_kv);
    if (need > ATTN_SCRATCH_BYTES)
        return fail(GQ_ERR_WORKSPACE, "flash_attn_ext_noalloc: this shape needs " + std::to_string(need) +
                                          " bytes of split partials, more than the " +
                                          std::to_string(ATTN_SCRATCH_BYTES) + "-byte static scratch");
    void* ptr = nullptr;
    if (need > 0) {
        const int rc = attn_scratch_init(&ptr);
        if (rc) return rc;
    }
    return attention(a, ptr, need, s);
}

}  // namespace gq
