// Probes used by the benchmark: a plain streaming read and a plain copy of a
// known number of bytes (the achievable HBM rate on the device and the
// calibration of the FETCH_SIZE / WRITE_SIZE counters), and matrix-core
// throughput loops (the achievable int8 / fp16 / fp64 MFMA rates, int8 in
// its 16x16x32, 32x32x32 and 16x16x64 forms).
#include "uq_device.h"
#include "uq_internal.h"
#include "../../include/uq.h"

#include <vector>

namespace uq {
namespace {

// Each workgroup reads one 28 KB chunk: seven non-temporal 16-byte loads per
// lane, lanes on consecutive pieces, all issued before the first is used; the
// dispatcher refills the CUs as workgroups retire (the access form of the
// lm_head matvecs). Of the read forms timed on MI355X (plain loads, LDS-DMA,
// 64-1024-thread workgroups, 12-48 KB chunks, persistent grid-stride loops)
// this one was the fastest at 131 MB, 249 MB and 1 GiB alike, so its rate is
// the achievable streaming-read ceiling the matvecs are compared with.
constexpr int PROBE_U = 7;
__global__ __launch_bounds__(256) void k_probe_read(const int4* __restrict__ src, int64_t n16, int* __restrict__ sink) {
    const int64_t b0 = (int64_t)blockIdx.x * (PROBE_U * 256) + threadIdx.x;
    int4 v[PROBE_U];
#pragma unroll
    for (int u = 0; u < PROBE_U; u++) {
        const int64_t j = b0 + 256 * u;
        v[u] = uq_ntload16(src + (j < n16 ? j : n16 - 1));
    }
    int acc = 0;
#pragma unroll
    for (int u = 0; u < PROBE_U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == 0x7fffffff) sink[blockIdx.x & 8191] = acc;  // keeps the loads live, never taken for zeroed memory
}

__global__ __launch_bounds__(256) void k_probe_copy(const int4* __restrict__ src, int4* __restrict__ dst, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

// MFMA throughput: every wave runs PC independent accumulator chains of
// `iters` dependent MFMAs on register operands. The sink store is never taken
// (the accumulators of small integer or zero products never reach the
// magic value) and only keeps the chains live.
typedef int pv4i __attribute__((ext_vector_type(4)));
typedef float pv4f __attribute__((ext_vector_type(4)));
typedef double pv4d __attribute__((ext_vector_type(4)));
typedef _Float16 pv8h __attribute__((ext_vector_type(8)));
constexpr int PC = 8;
__global__ __launch_bounds__(256) void k_probe_mfma_i8(int iters, int* __restrict__ sink) {
    const long a = (long)(threadIdx.x & 7), b = (long)((threadIdx.x >> 3) & 7);
    pv4i c[PC];
#pragma unroll
    for (int k = 0; k < PC; k++) c[k] = pv4i{0, 0, 0, 0};
    for (int i = 0; i < iters; i++)
#pragma unroll
        for (int k = 0; k < PC; k++) c[k] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c[k], 0, 0, 0);
    int s = 0;
#pragma unroll
    for (int k = 0; k < PC; k++) s += c[k][0] + c[k][1] + c[k][2] + c[k][3];
    if (s == 0x7fffffff) sink[blockIdx.x] = s;
}
// gfx950's K = 32 int8 form on 32 x 32 tiles (v_mfma_i32_32x32x32_i8, one
// 32-value block per instruction) and the K = 64 form on 16 x 16 tiles
// (v_mfma_i32_16x16x64_i8, two blocks): 16-byte operands per lane.
typedef int pv16i __attribute__((ext_vector_type(16)));
__global__ __launch_bounds__(256) void k_probe_mfma_i8_32x32(int iters, int* __restrict__ sink) {
    const pv4i a = {(int)(threadIdx.x & 7), 1, 2, 3}, b = {3, 2, 1, (int)((threadIdx.x >> 3) & 7)};
    pv16i c[PC / 2];
#pragma unroll
    for (int k = 0; k < PC / 2; k++)
#pragma unroll
        for (int r = 0; r < 16; r++) c[k][r] = 0;
    for (int i = 0; i < iters; i++)
#pragma unroll
        for (int k = 0; k < PC / 2; k++) c[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[k], 0, 0, 0);
    int s = 0;
#pragma unroll
    for (int k = 0; k < PC / 2; k++) s += c[k][0] + c[k][5] + c[k][10] + c[k][15];
    if (s == 0x7fffffff) sink[blockIdx.x] = s;
}
__global__ __launch_bounds__(256) void k_probe_mfma_i8_16x16x64(int iters, int* __restrict__ sink) {
    const pv4i a = {(int)(threadIdx.x & 7), 1, 2, 3}, b = {3, 2, 1, (int)((threadIdx.x >> 3) & 7)};
    pv4i c[PC];
#pragma unroll
    for (int k = 0; k < PC; k++) c[k] = pv4i{0, 0, 0, 0};
    for (int i = 0; i < iters; i++)
#pragma unroll
        for (int k = 0; k < PC; k++) c[k] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c[k], 0, 0, 0);
    int s = 0;
#pragma unroll
    for (int k = 0; k < PC; k++) s += c[k][0] + c[k][1] + c[k][2] + c[k][3];
    if (s == 0x7fffffff) sink[blockIdx.x] = s;
}
__global__ __launch_bounds__(256) void k_probe_mfma_f16(int iters, int* __restrict__ sink) {
    const _Float16 x = (_Float16)(float)(threadIdx.x & 3);
    const pv8h a = {x, x, x, x, x, x, x, x}, b = a;
    pv4f c[PC];
#pragma unroll
    for (int k = 0; k < PC; k++) c[k] = pv4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < iters; i++)
#pragma unroll
        for (int k = 0; k < PC; k++) c[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c[k], 0, 0, 0);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < PC; k++) s += c[k][0] + c[k][1] + c[k][2] + c[k][3];
    if (s == -1.0f) sink[blockIdx.x] = 1;
}
__global__ __launch_bounds__(256) void k_probe_mfma_f64(int iters, int* __restrict__ sink) {
    const double a = (double)(threadIdx.x & 3), b = (double)((threadIdx.x >> 2) & 3);
    pv4d c[PC];
#pragma unroll
    for (int k = 0; k < PC; k++) c[k] = pv4d{0.0, 0.0, 0.0, 0.0};
    for (int i = 0; i < iters; i++)
#pragma unroll
        for (int k = 0; k < PC; k++) c[k] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c[k], 0, 0, 0);
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < PC; k++) s += c[k][0] + c[k][1] + c[k][2] + c[k][3];
    if (s == -1.0) sink[blockIdx.x] = 1;
}
// One wave per SIMD (one 256-thread workgroup per CU), 16 MFMAs per iteration
// on four accumulator chains (MFMA) and/or the VALU work the prefill kernels
// put beside them (VALU): for FP64, a fresh fp16 operand converted to double
// per MFMA (the attention kernels' K and V operands); for int8, convert, scale
// product and fma of 16 f32 accumulators plus an integer step (the prefill
// GEMM's per-block rescale). Timing both alone and together shows whether the
// two overlap on a SIMD.
template <bool MFMA, bool VALU>
__global__ __launch_bounds__(256) void k_probe_f64_1w(int iters, int* __restrict__ sink) {
    const int t = threadIdx.x;
    double qa[16];
#pragma unroll
    for (int i = 0; i < 16; i++) qa[i] = 1.0 + 0.001 * (double)(t + i);
    uint32_t kw[8];
#pragma unroll
    for (int i = 0; i < 8; i++) kw[i] = 0x3c003c00u ^ (((uint32_t)t * 2654435761u + (uint32_t)i) & 0x03ff03ffu);
    pv4d c[4];
#pragma unroll
    for (int k = 0; k < 4; k++) c[k] = pv4d{0.0, 0.0, 0.0, 0.0};
    double vs = 0.0;
    for (int it = 0; it < iters; it++) {
        double kd[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            if (VALU) {
                const uint16_t h = (uint16_t)(i & 1 ? kw[i >> 1] >> 16 : kw[i >> 1] & 0xffff);
                kd[i] = (double)(float)__builtin_bit_cast(_Float16, h);
            } else {
                kd[i] = qa[(i + 3) & 15];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (MFMA) {
#pragma unroll
            for (int i = 0; i < 16; i++) c[i & 3] = __builtin_amdgcn_mfma_f64_16x16x4f64(qa[i], kd[i], c[i & 3], 0, 0, 0);
        } else {
            vs = kd[it & 15];
        }
        __builtin_amdgcn_sched_barrier(0);
        if (VALU) {
#pragma unroll
            for (int i = 0; i < 8; i++) kw[i] = kw[i] * 1664525u + 1013904223u;
        }
    }
    const pv4d u = (c[0] + c[1]) + (c[2] + c[3]);
    if (u[0] + u[1] + u[2] + u[3] + vs == -1.0) sink[blockIdx.x] = 1;
}
template <bool MFMA, bool VALU>
__global__ __launch_bounds__(256) void k_probe_i8_1w(int iters, int* __restrict__ sink) {
    const int t = threadIdx.x;
    long a = ((long)t << 32) ^ (long)(t * 3), b = ((long)(t * 7) << 32) ^ (long)t;
    pv4i c[4];
#pragma unroll
    for (int k = 0; k < 4; k++) c[k] = pv4i{0, 0, 0, 0};
    float y[16], sx[16];
    int d[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        y[i] = 0.0f;
        sx[i] = 0.001f * (float)(t + i);
        d[i] = t + i;
    }
    float sw = 0.5f + 0.001f * (float)t;
    for (int it = 0; it < iters; it++) {
        if (MFMA) {
#pragma unroll
            for (int i = 0; i < 16; i++) c[i & 3] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c[i & 3], 0, 0, 0);
        }
        if (VALU) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                y[i] = __builtin_fmaf((float)d[i], sx[i] * sw, y[i]);
                d[i] += 3;
            }
            sw += 0.25f;
        }
        a += 1;
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) s += y[i];
    if (s + (float)(c[0][0] + c[1][1] + c[2][2] + c[3][3]) == -1.0f) sink[blockIdx.x] = 1;
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
    const unsigned grid = 8192, rgrid = (unsigned)((n16 + PROBE_U * 256 - 1) / (PROBE_U * 256));
    hipEvent_t e0, e1;
    UQ_CHECK_HIP(hipEventCreate(&e0));
    UQ_CHECK_HIP(hipEventCreate(&e1));
    hipLaunchKernelGGL(k_probe_read, dim3(rgrid), dim3(256), 0, s, a, n16, sink);
    UQ_CHECK_HIP(hipEventRecord(e0, s));
    for (int r = 0; r < reps; r++) hipLaunchKernelGGL(k_probe_read, dim3(rgrid), dim3(256), 0, s, a, n16, sink);
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

int uq_probe_mfma(int kind, double* tera_ops) {
    if (!uq_stream()) return set_error(ERR_ARG, "uq_init has not been called");
    if (kind < 0 || kind > 10 || !tera_ops) return set_error(ERR_ARG, "probe_mfma: kind 0..10");
    hipStream_t s = (hipStream_t)uq_stream();
    const bool f64 = kind >= 2 && kind <= 5, one_wave = kind >= 3 && kind <= 8;
    // ops per wave instruction: 2*16*16*32 (int8, fp16), 2*16*16*4 (fp64),
    // 2*32*32*32 and 2*16*16*64 (the K = 32 and K = 64 int8 forms)
    const double ops = f64 ? 2.0 * 16 * 16 * 4 : kind == 9 ? 2.0 * 32 * 32 * 32 : kind == 10 ? 2.0 * 16 * 16 * 64
                                                                                              : 2.0 * 16 * 16 * 32;
    const int iters = kind == 2 ? 256 : kind >= 3 && kind <= 5 ? 512 : kind >= 9 ? 1024 : 2048;
    // 16 waves per CU, or one wave per SIMD (16 MFMAs per iteration, not PC)
    const unsigned grid = (one_wave ? 1u : 4u) * (unsigned)cu_count();
    const int per_iter = one_wave ? 16 : kind == 9 ? PC / 2 : PC;
    int* sink = nullptr;
    UQ_CHECK_HIP(hipMalloc(&sink, 4 * (size_t)grid));
    auto launch = [&]() {
        switch (kind) {
        case 0: hipLaunchKernelGGL(k_probe_mfma_i8, dim3(grid), dim3(256), 0, s, iters, sink); break;
        case 1: hipLaunchKernelGGL(k_probe_mfma_f16, dim3(grid), dim3(256), 0, s, iters, sink); break;
        case 2: hipLaunchKernelGGL(k_probe_mfma_f64, dim3(grid), dim3(256), 0, s, iters, sink); break;
        case 3: hipLaunchKernelGGL((k_probe_f64_1w<true, false>), dim3(grid), dim3(256), 0, s, iters, sink); break;
        case 4: hipLaunchKernelGGL((k_probe_f64_1w<true, true>), dim3(grid), dim3(256), 0, s, iters, sink); break;
        case 5: hipLaunchKernelGGL((k_probe_f64_1w<false, true>), dim3(grid), dim3(256), 0, s, iters, sink); break;
        case 6: hipLaunchKernelGGL((k_probe_i8_1w<true, false>), dim3(grid), dim3(256), 0, s, iters, sink); break;
        case 7: hipLaunchKernelGGL((k_probe_i8_1w<true, true>), dim3(grid), dim3(256), 0, s, iters, sink); break;
        case 8: hipLaunchKernelGGL((k_probe_i8_1w<false, true>), dim3(grid), dim3(256), 0, s, iters, sink); break;
        case 9: hipLaunchKernelGGL(k_probe_mfma_i8_32x32, dim3(grid), dim3(256), 0, s, iters, sink); break;
        default: hipLaunchKernelGGL(k_probe_mfma_i8_16x16x64, dim3(grid), dim3(256), 0, s, iters, sink); break;
        }
    };
    hipEvent_t e0, e1;
    UQ_CHECK_HIP(hipEventCreate(&e0));
    UQ_CHECK_HIP(hipEventCreate(&e1));
    launch();
    const int reps = 5;
    UQ_CHECK_HIP(hipEventRecord(e0, s));
    for (int r = 0; r < reps; r++) launch();
    UQ_CHECK_HIP(hipEventRecord(e1, s));
    UQ_CHECK_HIP(hipEventSynchronize(e1));
    float ms = 0;
    UQ_CHECK_HIP(hipEventElapsedTime(&ms, e0, e1));
    const double instrs = (double)grid * 4 * iters * per_iter * reps;
    *tera_ops = instrs * ops / (ms / 1e3) / 1e12;
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipFree(sink);
    return OK;
}

}  // extern "C"
