// Workgroup-level building blocks of the decode kernels: double sums and
// float max over a workgroup, the residual + RMSNorm + block-32 quant of one
// activation vector by one 256-thread workgroup, and the greedy candidate rule
// (stable argmax: lowest id wins ties, any non-finite logit marks it bad).
#pragma once
#include "uq_device.h"
#include "uq_decode.h"

namespace uq {

constexpr int NQ_WG = 256;

// Sum of a double over the whole workgroup (WG threads, multiple of 64).
template <int WG>
__device__ inline double block_sum_d(double v, double* red) {
    v = uq_group_sum<64>(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < WG / 64; w++) t += red[w];
    return t;
}
template <int WG>
__device__ inline float block_max_f(float v, float* red) {
    v = uq_group_max<64>(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int w = 1; w < WG / 64; w++) t = fmaxf(t, red[w]);
    return t;
}


// Residual + RMSNorm + block-32 quant of a.dim values by one workgroup of WG
// threads (element i = j*WG + t, so each 32-block sits in half a wave), in two
// halves: norm_quant_load issues the raw loads (activations, residual, gamma
// or the embedding row) and nothing else, so a kernel can issue its weight
// loads after it and still have the prologue wait only for the activations
// (vector-memory counters drain in issue order); norm_quant_finish does the
// arithmetic. The quantized vector goes to q/s (LDS or global; scale b at
// s[b * sstride]); write_x stores the summed residual to a.x_out. Ends with a
// barrier.
// PER elements per thread: dim <= PER * WG.
template <int PER>
struct NqRegs {
    float x[PER], r[PER], g[PER];
    int e[PER];
    uint16_t d[PER];
};
template <int WG, int MAXD>
using NqRegsFor = NqRegs<(MAXD + WG - 1) / WG>;

template <int WG, int PER>
__device__ __forceinline__ void norm_quant_load(const NormQuantArgs& a, NqRegs<PER>& v) {
    const int t = threadIdx.x, D = a.dim;
    const uint32_t tok = a.embed_qs ? *a.token : 0u;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = j * WG + t;
        if (i < D) {
            if (a.embed_qs) {
                const int64_t row = (int64_t)tok;
                v.d[j] = a.embed_d[row * (D / 32) + i / 32];
                v.e[j] = a.embed_qs[row * D + i];
            } else {
                v.x[j] = a.x[i];
                v.r[j] = a.residual ? a.residual[i] : 0.0f;
            }
            v.g[j] = a.gamma[i];
        }
    }
}

template <int WG, int PER>
__device__ __forceinline__ void norm_quant_finish(const NormQuantArgs& a, const NqRegs<PER>& v, bool write_x,
                                                  int8_t* q, float* s, double* red, int sstride = 1) {
    const int t = threadIdx.x, D = a.dim;
    float xv[PER];
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = j * WG + t;
        if (i < D) {
            float x;
            if (a.embed_qs) x = uq_half(v.d[j]) * (float)v.e[j];
            else x = a.residual ? v.x[j] + v.r[j] : v.x[j];
            if (write_x && a.x_out) a.x_out[i] = x;
            xv[j] = x;
            const float sq = x * x;
            ss += (double)sq;
        }
    }
    ss = block_sum_d<WG>(ss, red);
    const float mean = (float)(ss / (double)D);
    const float scale = 1.0f / sqrtf(mean + a.eps);
    // uq_quant_lane for all PER blocks of a thread at once: block maxima, then
    // the divisions spread over each 32-lane group (D % 32 == 0, so a block's
    // lanes are all in range or all out of it; out-of-range blocks are
    // computed on zeros and not stored)
    float y[PER], am[PER], inv[PER], sc[(PER + 31) / 32];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = j * WG + t;
        const float tmp = (i < D ? xv[j] : 0.0f) * scale;
        y[j] = tmp * (i < D ? v.g[j] : 0.0f);
        am[j] = uq_group_max<32>(fabsf(y[j]));
    }
    uq_block_recips<PER, 32>(am, inv, sc);
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = j * WG + t;
        if (i < D) q[i] = (int8_t)uq_quant_code(y[j], inv[j]);
    }
    // lane r of a 32-lane group holds the scales of its blocks j = r, r + 32, ...
#pragma unroll
    for (int k = 0; k < (PER + 31) / 32; k++) {
        const int j = (t & 31) + 32 * k, i = j * WG + (t & ~31);
        if (j < PER && i < D) s[(i >> 5) * sstride] = sc[k];
    }
    __syncthreads();
}

// The same residual + RMSNorm + block-32 quant done by ONE wave, for kernels
// whose other waves stream weights meanwhile, in two halves: issue() pulls the
// raw vectors (x, residual, gamma) into LDS staging by DMA (the embedding row
// into registers), so they hold no VGPRs while in flight; finish() waits for
// them and computes, with the sum of squares as a wave butterfly (no
// workgroup barrier). A kernel puts a barrier between the two halves and its
// weight loads after it, so that these loads enter the CU's memory queue
// ahead of the weight stream. Element i = 256*j + 4*lane + c, so a 32-block is
// 8 lanes. Requires dim % 32 == 0 and dim <= 256*NC; lx/lr/lg hold 256*NC
// floats each. The quantized vector goes to q (int8) and s (one f32 per block)
// in LDS; the caller's barrier publishes it.
template <int NC>
struct NormQuantWave {
    uint32_t e[NC];
    uint16_t d[NC];

    __device__ __forceinline__ void issue(const NormQuantArgs& a, float* lx, float* lr, float* lg) {
        const int lane = threadIdx.x & 63, D = a.dim;
        if (a.embed_qs) {
            const int64_t row = (int64_t)*a.token;
#pragma unroll
            for (int j = 0; j < NC; j++) {
                const int i = 256 * j + 4 * lane, ic = i < D ? i : D - 4;
                e[j] = *(const uint32_t*)(a.embed_qs + row * D + ic);
                d[j] = a.embed_d[row * (D / 32) + ic / 32];
                uq_lds_load16(a.gamma + ic, lg + 256 * j);
            }
        } else {
#pragma unroll
            for (int j = 0; j < NC; j++) {
                const int i = 256 * j + 4 * lane, ic = i < D ? i : D - 4;
                uq_lds_load16(a.x + ic, lx + 256 * j);
                if (a.residual) uq_lds_load16(a.residual + ic, lr + 256 * j);
                uq_lds_load16(a.gamma + ic, lg + 256 * j);
            }
        }
    }

    __device__ __forceinline__ void finish(const NormQuantArgs& a, bool write_x, const float* lx, const float* lr,
                                           const float* lg, int8_t* q, float* s) {
        const int lane = threadIdx.x & 63, D = a.dim;
        uq_wait_vm0();
        asm volatile("" ::: "memory");
        float xv[NC][4];
        double s4[4] = {0.0, 0.0, 0.0, 0.0};  // four chains of exact double terms
#pragma unroll
        for (int j = 0; j < NC; j++) {
            const int i = 256 * j + 4 * lane;
            if (a.embed_qs) {
                const float dd = uq_half(d[j]);
#pragma unroll
                for (int c = 0; c < 4; c++) xv[j][c] = dd * (float)(int8_t)(e[j] >> (8 * c));
            } else {
                const float4 xx = ((const float4*)lx)[64 * j + lane];
                xv[j][0] = xx.x;
                xv[j][1] = xx.y;
                xv[j][2] = xx.z;
                xv[j][3] = xx.w;
                if (a.residual) {
                    const float4 rr = ((const float4*)lr)[64 * j + lane];
                    xv[j][0] = xv[j][0] + rr.x;
                    xv[j][1] = xv[j][1] + rr.y;
                    xv[j][2] = xv[j][2] + rr.z;
                    xv[j][3] = xv[j][3] + rr.w;
                }
            }
            if (i < D) {
                if (write_x && a.x_out)
                    *(float4*)(a.x_out + i) = make_float4(xv[j][0], xv[j][1], xv[j][2], xv[j][3]);
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float sq = xv[j][c] * xv[j][c];
                    s4[c] += (double)sq;
                }
            } else {
#pragma unroll
                for (int c = 0; c < 4; c++) xv[j][c] = 0.0f;
            }
        }
        const double ss = uq_group_sum<64>((s4[0] + s4[1]) + (s4[2] + s4[3]));
        const float mean = (float)(ss / (double)D);
        const float scale = 1.0f / sqrtf(mean + a.eps);
        // the quant of uq_quant4_group8 for all NC blocks of a lane at once:
        // block maxima, then the divisions spread over each 8-lane group
        float y[NC][4], am[NC];
#pragma unroll
        for (int j = 0; j < NC; j++) {
            const float4 g4 = ((const float4*)lg)[64 * j + lane];
            const float gg[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float tmp = xv[j][c] * scale;
                y[j][c] = tmp * gg[c];
            }
            // lanes past dim hold zeros and form whole 8-lane groups
            const float m = fmaxf(fmaxf(fabsf(y[j][0]), fabsf(y[j][1])), fmaxf(fabsf(y[j][2]), fabsf(y[j][3])));
            am[j] = uq_group_max<8>(m);
        }
        float inv[NC], sc[(NC + 7) / 8];
        uq_block_recips<NC, 8>(am, inv, sc);
#pragma unroll
        for (int j = 0; j < NC; j++) {
            const int i = 256 * j + 4 * lane;
            uint32_t packed = 0;
#pragma unroll
            for (int c = 0; c < 4; c++) packed |= uq_quant_code(y[j][c], inv[j]) << (8 * c);
            if (i < D) *(uint32_t*)(q + i) = packed;
        }
        // lane 8g + r holds the scales of blocks j = r, r + 8, ...: block 8j + g of the row
#pragma unroll
        for (int k = 0; k < (NC + 7) / 8; k++) {
            const int j = (lane & 7) + 8 * k, i = 256 * j + 32 * (lane >> 3);
            if (j < NC && i < D) s[i >> 5] = sc[k];
        }
    }
};

// The same residual + RMSNorm + block-32 quant spread over all NW waves of a
// workgroup, for kernels whose weight stream is short (every wave can load
// and compute its share before its weights are needed): wave w takes the
// 256-value chunks w, w + NW, ... . issue() loads them into registers with
// plain loads, so a wave's weight loads issued afterwards keep exact vmcnt
// waits; finish() sums the wave's squares, meets the other waves' partial
// sums in LDS (part[NW], added in wave order in every wave) behind an LDS-only
// barrier, and quantizes its own chunks (divisions spread as in
// uq_block_recips). Per value the same operations as NormQuantWave. Every wave
// of the workgroup calls both halves; the caller's barrier publishes q / s
// (LDS or global; scale b at s[b * sstride]).
template <int NC, int NW>
struct NormQuantSplit {
    static constexpr int PC = (NC + NW - 1) / NW;  // chunks per wave, at most
    float4 xv[PC], rv[PC], gv[PC];
    uint32_t e[PC];
    uint16_t d[PC];

    __device__ __forceinline__ void issue(const NormQuantArgs& a) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, D = a.dim;
        const int64_t row = a.embed_qs ? (int64_t)(uint32_t)uq_sload((const int*)a.token) : 0;
#pragma unroll
        for (int k = 0; k < PC; k++) {
            const int c = wave + NW * k, cc = c < NC ? c : NC - 1;
            const int i = 256 * cc + 4 * lane, ic = i < D ? i : D - 4;
            if (a.embed_qs) {
                e[k] = *(const uint32_t*)(a.embed_qs + row * D + ic);
                d[k] = a.embed_d[row * (D / 32) + ic / 32];
            } else {
                xv[k] = *(const float4*)(a.x + ic);
                if (a.residual) rv[k] = *(const float4*)(a.residual + ic);
            }
            gv[k] = *(const float4*)(a.gamma + ic);
        }
    }

    __device__ __forceinline__ void finish(const NormQuantArgs& a, bool write_x, double* part, int8_t* q,
                                           float* s, int sstride = 1) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, D = a.dim;
        float x[PC][4];
        double s4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int k = 0; k < PC; k++) {
            const int c = wave + NW * k, i = 256 * c + 4 * lane;
            if (a.embed_qs) {
                const float dd = uq_half(d[k]);
#pragma unroll
                for (int m = 0; m < 4; m++) x[k][m] = dd * (float)(int8_t)(e[k] >> (8 * m));
            } else {
                x[k][0] = xv[k].x;
                x[k][1] = xv[k].y;
                x[k][2] = xv[k].z;
                x[k][3] = xv[k].w;
                if (a.residual) {
                    x[k][0] = x[k][0] + rv[k].x;
                    x[k][1] = x[k][1] + rv[k].y;
                    x[k][2] = x[k][2] + rv[k].z;
                    x[k][3] = x[k][3] + rv[k].w;
                }
            }
            if (c < NC && i < D) {
                if (write_x && a.x_out) *(float4*)(a.x_out + i) = make_float4(x[k][0], x[k][1], x[k][2], x[k][3]);
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    const float sq = x[k][m] * x[k][m];
                    s4[m] += (double)sq;
                }
            } else {
#pragma unroll
                for (int m = 0; m < 4; m++) x[k][m] = 0.0f;
            }
        }
        const double ws = uq_group_sum<64>((s4[0] + s4[1]) + (s4[2] + s4[3]));
        if (lane == 0) part[wave] = ws;
        // LDS-only barrier: the weight loads in flight are not waited for
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        double ss = part[0];
#pragma unroll
        for (int w = 1; w < NW; w++) ss += part[w];
        const float mean = (float)(ss / (double)D);
        const float scale = 1.0f / sqrtf(mean + a.eps);
        float y[PC][4], am[PC];
#pragma unroll
        for (int k = 0; k < PC; k++) {
            const float gg[4] = {gv[k].x, gv[k].y, gv[k].z, gv[k].w};
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const float tmp = x[k][m] * scale;
                y[k][m] = tmp * gg[m];
            }
            // lanes past dim hold zeros and form whole 8-lane groups
            const float mm = fmaxf(fmaxf(fabsf(y[k][0]), fabsf(y[k][1])), fmaxf(fabsf(y[k][2]), fabsf(y[k][3])));
            am[k] = uq_group_max<8>(mm);
        }
        float inv[PC], sc[(PC + 7) / 8];
        uq_block_recips<PC, 8>(am, inv, sc);
#pragma unroll
        for (int k = 0; k < PC; k++) {
            const int c = wave + NW * k, i = 256 * c + 4 * lane;
            uint32_t packed = 0;
#pragma unroll
            for (int m = 0; m < 4; m++) packed |= uq_quant_code(y[k][m], inv[k]) << (8 * m);
            if (c < NC && i < D) *(uint32_t*)(q + i) = packed;
        }
        // lane 8g + r holds the scale of chunk r (r < PC): block 8c + g of the row
#pragma unroll
        for (int kk = 0; kk < (PC + 7) / 8; kk++) {
            const int r = (lane & 7) + 8 * kk, c = wave + NW * r, i = 256 * c + 32 * (lane >> 3);
            if (r < PC && c < NC && i < D) s[(i >> 5) * sstride] = sc[kk];
        }
    }
};

template <int WG>
__device__ inline void norm_quant(const NormQuantArgs& a, bool write_x, int8_t* q, float* s, double* red,
                                  int sstride = 1) {
    NqRegsFor<WG, 4096> v;
    norm_quant_load<WG>(a, v);
    norm_quant_finish<WG>(a, v, write_x, q, s, red, sstride);
}

struct Cand {
    float v;
    int id;
    unsigned bad;
    unsigned pad;
};
__device__ __forceinline__ bool better(float a, int ai, float b, int bi) { return a > b || (a == b && ai < bi); }
__device__ inline void cand_reduce(float& v, int& id, unsigned& bad, float* vs, int* ids, unsigned* bs) {
    const int t = threadIdx.x;
    vs[t] = v;
    ids[t] = id;
    bs[t] = bad;
    __syncthreads();
    for (int d = blockDim.x / 2; d; d >>= 1) {
        if (t < d) {
            if (better(vs[t + d], ids[t + d], vs[t], ids[t])) {
                vs[t] = vs[t + d];
                ids[t] = ids[t + d];
            }
            bs[t] |= bs[t + d];
        }
        __syncthreads();
    }
    v = vs[0];
    id = ids[0];
    bad = bs[0];
}

}  // namespace uq
