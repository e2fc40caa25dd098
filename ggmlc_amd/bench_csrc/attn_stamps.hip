// Timestamped build of libgq's attention for the benchmark's measurement runs (linked into
// libgqbench.so only): the same source compiled with GQ_ATTN_STAMPS, in a namespace of its
// own so that none of its symbols interposes libgq's. k_attn_dec then records per-wave
// s_memrealtime stamps (event list at g_attn_stamps in attention.hip); everything else,
// including the launch plan, is libgq's code.
#define GQ_ATTN_STAMPS 1
#define gq gqstamp
#include "../csrc/attention.hip"

#include <string>

namespace gqstamp {

// the pieces of api.hip the attention code calls
static thread_local std::string g_err;
void set_error(const std::string& msg) { g_err = msg; }
int fail(int code, const std::string& msg) {
    set_error(msg);
    return code;
}
int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return GQ_OK;
    return fail(GQ_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}
bool option_attn_separate_merge() { return false; }

}  // namespace gqstamp
#undef gq

extern "C" {

const char* gqbench_attn_last_error(void) { return gqstamp::g_err.c_str(); }

/* Decode attention (gq_flash_attn_ext's contiguous path) through the timestamped build:
 * q [Hq][S][D] fp32 rows, K/V heads of n_kv rows of D fp16 (row stride D * 2 bytes, head
 * stride kv_head_bytes), mask [S][n_kv] fp16, dst [S][Hq][D] fp32; workspace as
 * gq_flash_attn_ext_workspace_size gives it. */
int gqbench_attn_stamped(const float* q, int64_t D, int64_t S, int64_t Hq, int64_t Hkv, const uint16_t* k,
                         const uint16_t* v, int64_t n_kv, int64_t kv_head_bytes, const uint16_t* mask, float scale,
                         float* dst, void* ws, size_t ws_bytes, void* stream) {
    gqstamp::AttnArgs a{};
    a.q = q;
    a.D = D;
    a.S = S;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.qnb1 = D * 4;
    a.qnb2 = S * D * 4;
    a.k = k;
    a.v = v;
    a.n_kv = n_kv;
    a.knb1 = a.vnb1 = D * 2;
    a.knb2 = a.vnb2 = kv_head_bytes;
    a.mask = mask;
    a.mnb1 = n_kv * 2;
    a.scale = scale;
    a.dst = dst;
    return gqstamp::attention(a, ws, ws_bytes, (hipStream_t)stream);
}

/* Copies the stamp array (gqbench_attn_stamp_slots() 64-bit words) to host memory and
 * clears it on the device. */
int gqbench_attn_stamp_slots(void) { return gqstamp::STAMP_SLOTS; }
int gqbench_attn_stamps_take(unsigned long long* host) {
    void* p = nullptr;
    int rc = gqstamp::check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(gqstamp::g_attn_stamps)), "stamp symbol");
    if (rc) return rc;
    const size_t n = sizeof(unsigned long long) * gqstamp::STAMP_SLOTS;
    rc = gqstamp::check_hip(hipMemcpy(host, p, n, hipMemcpyDeviceToHost), "stamp copy");
    if (rc) return rc;
    return gqstamp::check_hip(hipMemset(p, 0, n), "stamp clear");
}

}  // extern "C"
