// Bandwidth probes used by the benchmark: a plain streaming read and a plain
// copy of a known number of bytes. They give the achievable HBM rate on the box
// and the calibration of the FETCH_SIZE / WRITE_SIZE counters.
#include "uq_internal.h"
#include "../../include/uq.h"

#include <vector>

namespace uq {
namespace {

__global__ __launch_bounds__(256) void k_probe_read(const int4* __restrict__ src, int64_t n16, int* __restrict__ sink) {
    int acc = 0;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += 4 * stride) {
        int4 v0 = src[i];
        int4 v1 = i + stride < n16 ? src[i + stride] : make_int4(0, 0, 0, 0);
        int4 v2 = i + 2 * stride < n16 ? src[i + 2 * stride] : make_int4(0, 0, 0, 0);
        int4 v3 = i + 3 * stride < n16 ? src[i + 3 * stride] : make_int4(0, 0, 0, 0);
        acc ^= v0.x ^ v0.y ^ v0.z ^ v0.w ^ v1.x ^ v1.y ^ v1.z ^ v1.w;
        acc ^= v2.x ^ v2.y ^ v2.z ^ v2.w ^ v3.x ^ v3.y ^ v3.z ^ v3.w;
    }
    if (acc == 0x7fffffff) sink[blockIdx.x] = acc;  // keeps the loads live, never taken for zeroed memory
}

__global__ __launch_bounds__(256) void k_probe_copy(const int4* __restrict__ src, int4* __restrict__ dst, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

}  // namespace
}  // namespace uq

using namespace uq;

extern "C" {

int uq_probe_bandwidth(int64_t bytes, int reps, double* read_gbs, double* copy_gbs) {
    if (!uq_stream()) return set_error(ERR_ARG, "uq_init has not been called");
    if (bytes < (1 << 20) || reps <= 0) return set_error(ERR_ARG, "probe_bandwidth: bytes >= 1 MiB, reps > 0");
    hipStream_t s = (hipStream_t)uq_stream();
    const int64_t n16 = bytes / 16;
    int4 *a = nullptr, *b = nullptr;
    int* sink = nullptr;
    UQ_CHECK_HIP(hipMalloc(&a, n16 * 16));
    UQ_CHECK_HIP(hipMalloc(&b, n16 * 16));
    UQ_CHECK_HIP(hipMalloc(&sink, 4 * 8192));
    UQ_CHECK_HIP(hipMemsetAsync(a, 0, n16 * 16, s));
    const unsigned grid = 8192;
    hipEvent_t e0, e1;
    UQ_CHECK_HIP(hipEventCreate(&e0));
    UQ_CHECK_HIP(hipEventCreate(&e1));
    hipLaunchKernelGGL(k_probe_read, dim3(grid), dim3(256), 0, s, a, n16, sink);
    UQ_CHECK_HIP(hipEventRecord(e0, s));
    for (int r = 0; r < reps; r++) hipLaunchKernelGGL(k_probe_read, dim3(grid), dim3(256), 0, s, a, n16, sink);
    UQ_CHECK_HIP(hipEventRecord(e1, s));
    UQ_CHECK_HIP(hipEventSynchronize(e1));
    float ms = 0;
    UQ_CHECK_HIP(hipEventElapsedTime(&ms, e0, e1));
    if (read_gbs) *read_gbs = (double)n16 * 16 * reps / (ms / 1e3) / 1e9;
    hipLaunchKernelGGL(k_probe_copy, dim3(grid), dim3(256), 0, s, a, b, n16);
    UQ_CHECK_HIP(hipEventRecord(e0, s));
    for (int r = 0; r < reps; r++) hipLaunchKernelGGL(k_probe_copy, dim3(grid), dim3(256), 0, s, a, b, n16);
    UQ_CHECK_HIP(hipEventRecord(e1, s));
    UQ_CHECK_HIP(hipEventSynchronize(e1));
    UQ_CHECK_HIP(hipEventElapsedTime(&ms, e0, e1));
    if (copy_gbs) *copy_gbs = (double)n16 * 16 * 2 * reps / (ms / 1e3) / 1e9;  // read + write bytes
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipFree(a);
    hipFree(b);
    hipFree(sink);
    return OK;
}

}  // extern "C"
