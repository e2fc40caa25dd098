// Timestamped build of libgq's int8 GEMM for the benchmark's measurement runs (linked into
// libgqbench.so only): the same source compiled with GQ_GEMM_STAMPS, in a namespace of its
// own so that none of its symbols interposes libgq's. k_gemm_i8's quantized-SWIGLU launches
// then record per-wave s_memrealtime stamps (event list at g_gemm_stamps in gemm_i8.hip);
// everything else, including the launch plan, is libgq's code.
#define GQ_GEMM_STAMPS 1
#define gq gqgstamp
#include "../csrc/gemm_i8.hip"

#include <string>

namespace gqgstamp {

// the pieces of api.hip the GEMM code calls
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
bool option_gemm_i8_ring() { return false; }

}  // namespace gqgstamp
#undef gq

extern "C" {

const char* gqbench_gemm_last_error(void) { return gqgstamp::g_err.c_str(); }

/* The gate|up product with SWIGLU and the quantized rows (gq_mul_mat_fused with swiglu and
 * out_q8 on the int8 path) through the timestamped build: W [N][K] Q8_0 / Q4_0 rows, act
 * the M rows in act_prep_i8's layout, dst [M][N/2] fp32 (row stride ldd floats, may be
 * null), q8 the quantized SWIGLU rows (K = N/2 layout). */
int gqbench_gemm_i8_glu_stamped(int type, const void* W, int64_t N, int64_t K, const void* act, int64_t M,
                                float* dst, int64_t ldd, void* q8, void* stream) {
    gqgstamp::I8Epi e{};
    e.glu = 1;
    e.pair_lo = ~(int64_t)0;
    e.pair_h = N / 2;
    e.q8 = static_cast<uint8_t*>(q8);
    return gqgstamp::gemm_i8(type, static_cast<const uint8_t*>(W), N, K, static_cast<const uint8_t*>(act), M, dst,
                             ldd, (hipStream_t)stream, nullptr, &e);
}

/* Copies the stamp array (gqbench_gemm_stamp_slots() 64-bit words) to host memory and
 * clears it on the device. */
int gqbench_gemm_stamp_slots(void) { return gqgstamp::GSTAMP_SLOTS; }
int gqbench_gemm_stamps_take(unsigned long long* host) {
    void* p = nullptr;
    int rc = gqgstamp::check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(gqgstamp::g_gemm_stamps)), "stamp symbol");
    if (rc) return rc;
    const size_t n = sizeof(unsigned long long) * gqgstamp::GSTAMP_SLOTS;
    rc = gqgstamp::check_hip(hipMemcpy(host, p, n, hipMemcpyDeviceToHost), "stamp copy");
    if (rc) return rc;
    return gqgstamp::check_hip(hipMemset(p, 0, n), "stamp clear");
}

}  // extern "C"
