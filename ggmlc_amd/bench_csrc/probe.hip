// Streaming-read probe of the benchmark (libgqbench.so, loaded by bench.py only; not
// part of libgq's ABI): reads a buffer once with coalesced 16-byte nontemporal loads
// (the access pattern of the GEMV weight stream) so a benchmark can state the HBM read
// bandwidth this device actually sustains next to the datasheet peak.
#include "common.h"

namespace {

using gq::ld_nt16;

__global__ __launch_bounds__(256) void k_read_probe(const uint4* __restrict__ p, int64_t n16,
                                                    uint32_t* __restrict__ sink) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = ld_nt16(p + i);
        const uint4 b = ld_nt16(p + i + stride);
        const uint4 c = ld_nt16(p + i + 2 * stride);
        const uint4 d = ld_nt16(p + i + 3 * stride);
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += stride) {
        const uint4 a = ld_nt16(p + i);
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads alive; practically never taken
}

}  // namespace

// Reads `bytes` (16-byte aligned) of p once with `grid` workgroups of 256 threads; sink: a
// device uint32 that is (practically) never written. Returns 0, or a HIP error code.
extern "C" int gqbench_stream_read_grid(const void* p, size_t bytes, int grid, uint32_t* sink, hipStream_t s) {
    if (grid < 1) return (int)hipErrorInvalidValue;
    const int64_t n16 = (int64_t)(bytes / 16);
    hipLaunchKernelGGL(k_read_probe, dim3((unsigned)grid), dim3(256), 0, s, reinterpret_cast<const uint4*>(p), n16,
                       sink);
    return (int)hipGetLastError();
}

// The same with 8 workgroups per CU (the grid of the bandwidth calibration)
extern "C" int gqbench_stream_read(const void* p, size_t bytes, uint32_t* sink, hipStream_t s) {
    int dev = 0, ncu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return (int)e;
    return gqbench_stream_read_grid(p, bytes, ncu * 8, sink, s);
}
