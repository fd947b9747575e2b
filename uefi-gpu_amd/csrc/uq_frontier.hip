// fp32-activation reader of the reference's frontier backend on gfx950: the
// seven GGUF kinds of its frontier model (F32, BF16, Q8_0, Q6_K, IQ3_XXS,
// IQ4_NL, IQ4_XS), a bit-exact dequant, and y = W x with fp32 x for one
// weight or for a job table of many weights in one launch.
//
// Replaces frontier_dequant / frontier_matvec / frontier_multi_matvec
// (driver/kernels/frontier_quant.cu:12-93) and their CPU definition
// dequantize (driver/src/frontier_core.rs:73-106), behind Weights::linear and
// Weights::batch (driver/src/frontier_forward.rs:14-28, frontier_backend.rs).
//
// Arithmetic. Every decoded weight of these kinds is an integer code times an
// f32 block scale that is itself an exact product (fp16 d times a small
// integer, or a power-of-two fraction of one), so sum_i w_i x_i equals
// sum over scale groups of scale * sum(code * x) exactly. The kernels form
// each code * x in double (exact), sum a scale group in double, multiply by
// the exact scale in double, add the groups of a lane in unit order, reduce
// the lanes of a row in double and round to f32 once: the oracle's exact
// double sum up to ~2^-50 relative, so both agree bit for bit except in rare
// rounding-boundary cases (<= 1 ulp). The single-weight and job-table forms
// run the same kernel, so they agree bit for bit always.
//
// Device layouts (split by the verified upload in uq_runtime.hip): a body
// plane of 16-byte aligned units per row, a per-block fp16 scale plane, and an
// aux plane (IQ4_XS block head, Q6_K scales in unit order); see frontier_layout.
#include "uq_device.h"
#include "uq_internal.h"
#include "../../include/uq.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

namespace uq {
namespace {

// IQ4_NL / IQ4_XS code book (frontier_core.rs:67) and the IQ3_XXS grid
// (frontier_tables.rs:2-35, ggml's iq3xxs_grid): data of the format, from
// ggml (MIT licence, third_party/LICENSE.ggml).
__constant__ __attribute__((aligned(16))) int8_t c_iq4[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
__constant__ uint32_t c_iq3_grid[256] = {
    0x04040404u, 0x04040414u, 0x04040424u, 0x04040c0cu, 0x04040c1cu, 0x04040c3eu, 0x04041404u, 0x04041414u,
    0x04041c0cu, 0x04042414u, 0x04043e1cu, 0x04043e2cu, 0x040c040cu, 0x040c041cu, 0x040c0c04u, 0x040c0c14u,
    0x040c140cu, 0x040c142cu, 0x040c1c04u, 0x040c1c14u, 0x040c240cu, 0x040c2c24u, 0x040c3e04u, 0x04140404u,
    0x04140414u, 0x04140424u, 0x04140c0cu, 0x04141404u, 0x04141414u, 0x04141c0cu, 0x04141c1cu, 0x04141c3eu,
    0x04142c0cu, 0x04142c3eu, 0x04143e2cu, 0x041c040cu, 0x041c043eu, 0x041c0c04u, 0x041c0c14u, 0x041c142cu,
    0x041c3e04u, 0x04240c1cu, 0x04241c3eu, 0x04242424u, 0x04242c3eu, 0x04243e1cu, 0x04243e2cu, 0x042c040cu,
    0x042c043eu, 0x042c1c14u, 0x042c2c14u, 0x04341c2cu, 0x04343424u, 0x043e0c04u, 0x043e0c24u, 0x043e0c34u,
    0x043e241cu, 0x043e340cu, 0x0c04040cu, 0x0c04041cu, 0x0c040c04u, 0x0c040c14u, 0x0c04140cu, 0x0c04141cu,
    0x0c041c04u, 0x0c041c14u, 0x0c041c24u, 0x0c04243eu, 0x0c042c04u, 0x0c0c0404u, 0x0c0c0414u, 0x0c0c0c0cu,
    0x0c0c1404u, 0x0c0c1414u, 0x0c14040cu, 0x0c14041cu, 0x0c140c04u, 0x0c140c14u, 0x0c14140cu, 0x0c141c04u,
    0x0c143e14u, 0x0c1c0404u, 0x0c1c0414u, 0x0c1c1404u, 0x0c1c1c0cu, 0x0c1c2434u, 0x0c1c3434u, 0x0c24040cu,
    0x0c24042cu, 0x0c242c04u, 0x0c2c1404u, 0x0c2c1424u, 0x0c2c2434u, 0x0c2c3e0cu, 0x0c34042cu, 0x0c3e1414u,
    0x0c3e2404u, 0x14040404u, 0x14040414u, 0x14040c0cu, 0x14040c1cu, 0x14041404u, 0x14041414u, 0x14041434u,
    0x14041c0cu, 0x14042414u, 0x140c040cu, 0x140c041cu, 0x140c042cu, 0x140c0c04u, 0x140c0c14u, 0x140c140cu,
    0x140c1c04u, 0x140c341cu, 0x140c343eu, 0x140c3e04u, 0x14140404u, 0x14140414u, 0x14140c0cu, 0x14140c3eu,
    0x14141404u, 0x14141414u, 0x14141c3eu, 0x14142404u, 0x14142c2cu, 0x141c040cu, 0x141c0c04u, 0x141c0c24u,
    0x141c3e04u, 0x141c3e24u, 0x14241c2cu, 0x14242c1cu, 0x142c041cu, 0x142c143eu, 0x142c240cu, 0x142c3e24u,
    0x143e040cu, 0x143e041cu, 0x143e0c34u, 0x143e242cu, 0x1c04040cu, 0x1c040c04u, 0x1c040c14u, 0x1c04140cu,
    0x1c04141cu, 0x1c042c04u, 0x1c04342cu, 0x1c043e14u, 0x1c0c0404u, 0x1c0c0414u, 0x1c0c1404u, 0x1c0c1c0cu,
    0x1c0c2424u, 0x1c0c2434u, 0x1c14040cu, 0x1c14041cu, 0x1c140c04u, 0x1c14142cu, 0x1c142c14u, 0x1c143e14u,
    0x1c1c0c0cu, 0x1c1c1c1cu, 0x1c241c04u, 0x1c24243eu, 0x1c243e14u, 0x1c2c0404u, 0x1c2c0434u, 0x1c2c1414u,
    0x1c2c2c2cu, 0x1c340c24u, 0x1c341c34u, 0x1c34341cu, 0x1c3e1c1cu, 0x1c3e3404u, 0x24040424u, 0x24040c3eu,
    0x24041c2cu, 0x24041c3eu, 0x24042c1cu, 0x24042c3eu, 0x240c3e24u, 0x24141404u, 0x24141c3eu, 0x24142404u,
    0x24143404u, 0x24143434u, 0x241c043eu, 0x241c242cu, 0x24240424u, 0x24242c0cu, 0x24243424u, 0x242c142cu,
    0x242c241cu, 0x242c3e04u, 0x243e042cu, 0x243e0c04u, 0x243e0c14u, 0x243e1c04u, 0x2c040c14u, 0x2c04240cu,
    0x2c043e04u, 0x2c0c0404u, 0x2c0c0434u, 0x2c0c1434u, 0x2c0c2c2cu, 0x2c140c24u, 0x2c141c14u, 0x2c143e14u,
    0x2c1c0414u, 0x2c1c2c1cu, 0x2c240c04u, 0x2c24141cu, 0x2c24143eu, 0x2c243e14u, 0x2c2c0414u, 0x2c2c1c0cu,
    0x2c342c04u, 0x2c3e1424u, 0x2c3e2414u, 0x34041424u, 0x34042424u, 0x34042434u, 0x34043424u, 0x340c140cu,
    0x340c340cu, 0x34140c3eu, 0x34143424u, 0x341c1c04u, 0x341c1c34u, 0x34242424u, 0x342c042cu, 0x342c2c14u,
    0x34341c1cu, 0x343e041cu, 0x343e140cu, 0x3e04041cu, 0x3e04042cu, 0x3e04043eu, 0x3e040c04u, 0x3e041c14u,
    0x3e042c14u, 0x3e0c1434u, 0x3e0c2404u, 0x3e140c14u, 0x3e14242cu, 0x3e142c14u, 0x3e1c0404u, 0x3e1c0c2cu,
    0x3e1c1c1cu, 0x3e1c3404u, 0x3e24140cu, 0x3e24240cu, 0x3e2c0404u, 0x3e2c0414u, 0x3e2c1424u, 0x3e341c04u,
};

constexpr int FWG = 256;
constexpr int FL_WG = 512;  // workgroup of the linear kernel

// ---------------------------------------------------------------- dequant
// One value per thread from the GGUF bytes, the formulas and f32 multiply
// order of dequantize (frontier_core.rs:73-106).
__device__ __forceinline__ uint32_t rd16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
__device__ __forceinline__ uint32_t rd32(const uint8_t* p) { return rd16(p) | (rd16(p + 2) << 16); }

__device__ float dequant_value(uint32_t kind, const uint8_t* in, int64_t i) {
    switch (kind) {
    case KIND_F32: return uq_bits_f(rd32(in + 4 * i));
    case KIND_BF16: return uq_bits_f(rd16(in + 2 * i) << 16);
    case KIND_Q8_0: {
        const uint8_t* p = in + (i / 32) * 34;
        return uq_half((uint16_t)rd16(p)) * (float)(int8_t)p[2 + i % 32];
    }
    case KIND_IQ4_NL: {
        const uint8_t* p = in + (i / 32) * 18;
        const int j = (int)(i % 32), q = (p[2 + j % 16] >> (4 * (j / 16))) & 15;
        return uq_half((uint16_t)rd16(p)) * (float)c_iq4[q];
    }
    case KIND_IQ4_XS: {
        const uint8_t* p = in + (i / 256) * 136;
        const int j = (int)(i % 256), sb = j / 32;
        const int sc = ((p[4 + sb / 2] >> (4 * (sb % 2))) & 15) | (((rd16(p + 2) >> (2 * sb)) & 3) << 4);
        const int q = (p[8 + sb * 16 + j % 16] >> (4 * ((j % 32) / 16))) & 15;
        return (uq_half((uint16_t)rd16(p)) * (float)(sc - 32)) * (float)c_iq4[q];
    }
    case KIND_Q6_K: {
        const uint8_t* p = in + (i / 256) * 210;
        const int j = (int)(i % 256), sub = j / 128, l = j % 32, g = (j % 128) / 32;
        const int lo = p[sub * 64 + l + (g % 2) * 32], hi = p[128 + sub * 32 + l];
        const int q = (((lo >> (4 * (g / 2))) & 15) | (((hi >> (2 * g)) & 3) << 4)) - 32;
        const int sc = (int8_t)p[192 + sub * 8 + l / 16 + g * 2];
        return (uq_half((uint16_t)rd16(p + 208)) * (float)sc) * (float)q;
    }
    case KIND_IQ3_XXS: {
        const uint8_t* p = in + (i / 256) * 98;
        const int j = (int)(i % 256), sb = j / 32, g = (j % 32) / 8;
        const uint32_t aux = rd32(p + 66 + sb * 4), s7 = (aux >> (7 * g)) & 127;
        const uint32_t sg = s7 | ((uint32_t)(__popc(s7) & 1) << 7);
        const int idx = p[2 + sb * 8 + g * 2 + (j % 8) / 4];
        const uint32_t q = (c_iq3_grid[idx] >> (8 * (j % 4))) & 255;
        const float scale = uq_half((uint16_t)rd16(p)) * (0.5f + (float)(aux >> 28)) * 0.5f;
        return (scale * (float)q) * ((sg & (1u << (j % 8))) ? -1.0f : 1.0f);
    }
    }
    return __builtin_nanf("");
}

__global__ __launch_bounds__(FWG) void k_dequant(const uint8_t* __restrict__ in, float* __restrict__ out, uint32_t kind,
                                                 int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * FWG + threadIdx.x; i < n; i += (int64_t)gridDim.x * FWG)
        out[i] = dequant_value(kind, in, i);
}

// ---------------------------------------------------------------- layout repack / verify
// Byte map of one GGUF block into the planes: map[o] = plane << 12 | offset
// within that plane's block (plane 0 body, 1 aux, 2 fp16 scale).
struct MapArgs {
    uint16_t map[256];
    int32_t block_bytes, plane_bytes[3];
};

__global__ __launch_bounds__(FWG) void k_layout_repack(const uint8_t* __restrict__ src, int64_t blocks, MapArgs a,
                                                       uint8_t* p0, uint8_t* p1, uint8_t* p2) {
    const int64_t total = blocks * a.block_bytes;
    for (int64_t i = (int64_t)blockIdx.x * FWG + threadIdx.x; i < total; i += (int64_t)gridDim.x * FWG) {
        const int64_t b = i / a.block_bytes;
        const int o = (int)(i - b * a.block_bytes), e = a.map[o], pl = e >> 12, off = e & 0xfff;
        uint8_t* dst = pl == 0 ? p0 : (pl == 1 ? p1 : p2);
        dst[b * a.plane_bytes[pl] + off] = src[i];
    }
}

__global__ __launch_bounds__(FWG) void k_layout_verify(const uint8_t* __restrict__ src, int64_t blocks, MapArgs a,
                                                       const uint8_t* p0, const uint8_t* p1, const uint8_t* p2,
                                                       unsigned* bad) {
    const int64_t total = blocks * a.block_bytes;
    unsigned miss = 0;
    for (int64_t i = (int64_t)blockIdx.x * FWG + threadIdx.x; i < total; i += (int64_t)gridDim.x * FWG) {
        const int64_t b = i / a.block_bytes;
        const int o = (int)(i - b * a.block_bytes), e = a.map[o], pl = e >> 12, off = e & 0xfff;
        const uint8_t* dst = pl == 0 ? p0 : (pl == 1 ? p1 : p2);
        miss += dst[b * a.plane_bytes[pl] + off] != src[i];
    }
    if (miss) atomicAdd(bad, miss);
}

// ---------------------------------------------------------------- fp32-x matvec
// Job of the launch (the FrontierJob of frontier_quant.cu:71-78 with the
// planes of an uploaded weight): rows [0, m) of one weight times x.
struct FJob {
    const uint8_t* body;  // row r's units start at body + r * pitch
    const uint8_t* aux;
    const uint16_t* d;
    const float* x;
    float* y;
    int64_t m, pitch;
    int32_t kind, n;
    int32_t wg0, wgs;  // first workgroup of the job, workgroups of the job
};

// ---- exact integer form of x
// Each 32-block of x is staged in LDS as integers X_j with x_j = X_j *
// 2^(E - XSHIFT), E = max(biased exponent of max|x_j|, 1): X_j = m_j *
// 2^(e_j - E + 14) for the 24-bit significand m_j, |X_j| < 2^38, exact when
// every element lies within 2^14 of the block maximum (or its dropped low bits
// are zero). X_j is held as five balanced base-256 digits in five byte planes,
// so sum(code * X) over a block is five v_dot4 sums recombined exactly in
// double (|sum| < 2^51). A block that is not exact (wider range, or a
// non-finite value) is marked and its dots run in double from x itself.
constexpr int XSHIFT = 164, NLIMB = 5;

struct XStage {
    const uint32_t* limb;  // NLIMB planes of n/16 16-byte chunks (16 elements), in unit-major slots
    const int* bexp;       // per 32-block: E, or -1 when the block takes the double path
    const float* xg;       // x in global memory (double path)
    const float* xf;       // F32 / BF16 weights: x as f32 in LDS
    int n4;                // n / 4: dwords per plane
};

// Digit chunks are held unit-major: chunk k (elements 16k..16k+15) of the
// job's kind sits in slot pos * NU + u, u its unit and pos its place in the
// unit (NU units per row), so the lanes of a row group, which own
// consecutive units, read consecutive 16-byte slots.
__device__ __forceinline__ int chunk_slot(uint32_t kind, int k, int n) {
    switch (kind) {
    case KIND_Q6_K: {  // unit 4s + 2sub + h holds chunks 16s + 8sub + 2g + h, place g
        const int u = 4 * (k >> 4) + 2 * ((k >> 3) & 1) + (k & 1);
        return ((k >> 1) & 3) * (n / 64) + u;
    }
    case KIND_IQ3_XXS: return (k & 7) * (n / 128) + (k >> 3);
    default: return (k & 1) * (n / 32) + (k >> 1);  // Q8_0, IQ4_NL, IQ4_XS: 2 chunks per unit
    }
}

// sum(code * x) over NC chunks (4 dwords of packed signed codes each) in
// slots slot0, slot0 + sstride, ...; e0 = first element (32-block exponent,
// double path) and the chunks cover elements e0 + 16*c.
template <int NC>
__device__ __forceinline__ double seg_dot(const uint32_t (&c)[4 * NC], const XStage& xs, int e0, int slot0,
                                          int sstride) {
    const int E = xs.bexp[e0 >> 5];
    if (E >= 0) {
        int S[NLIMB];
#pragma unroll
        for (int l = 0; l < NLIMB; l++) {
            int a = 0;
#pragma unroll
            for (int ch = 0; ch < NC; ch++) {
                const uint4 p = ((const uint4*)xs.limb)[l * (xs.n4 >> 2) + slot0 + ch * sstride];
                a = uq_dot4((int)c[4 * ch + 0], (int)p.x, a);
                a = uq_dot4((int)c[4 * ch + 1], (int)p.y, a);
                a = uq_dot4((int)c[4 * ch + 2], (int)p.z, a);
                a = uq_dot4((int)c[4 * ch + 3], (int)p.w, a);
            }
            S[l] = a;
        }
        double t = (double)S[NLIMB - 1];
#pragma unroll
        for (int l = NLIMB - 2; l >= 0; l--) t = __builtin_fma(t, 256.0, (double)S[l]);
        return __builtin_ldexp(t, E - XSHIFT);
    }
    double s[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int q = 0; q < 4 * NC; q++)
#pragma unroll
        for (int k = 0; k < 4; k++)
            s[k] = __builtin_fma((double)(int)(int8_t)(uint8_t)(c[q] >> (8 * k)), (double)xs.xg[e0 + 4 * q + k], s[k]);
    return (s[0] + s[1]) + (s[2] + s[3]);
}

// Stages x of one job, 4 elements per thread (8 threads per 32-block): the
// block's exponent from the 8-lane max of |x|, each X_j, and its five digits
// packed 4 elements per dword into the five planes (byte l of X_j + 0x80 in
// every digit position, minus 0x80: balanced digits in [-128, 127]).
__device__ void stage_x(const float* __restrict__ x, int n, uint32_t kind, uint32_t* limb, int* bexp) {
    const int n4 = n / 4;
    for (int q = threadIdx.x; q < ((n4 + 7) & ~7); q += (int)blockDim.x) {
        // q < n4 for the whole 8-lane group or for none of it (n % 32 == 0)
        if (q < n4) {
            const float4 v4 = ((const float4*)x)[q];
            const float v[4] = {v4.x, v4.y, v4.z, v4.w};
            float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
            amax = uq_group_max<8>(amax);
            int E = (int)(__builtin_bit_cast(uint32_t, amax) >> 23);
            bool ok = E < 255 && !(amax != amax);
            E = E < 1 ? 1 : E;
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t bits = __builtin_bit_cast(uint32_t, v[k]);
                const int eb = (int)((bits >> 23) & 255);
                uint32_t m = bits & 0x7FFFFFu;
                if (eb) m |= 0x800000u;
                const int sh = (eb < 1 ? 1 : eb) - E + 14;
                int64_t X = 0;
                if (eb == 255) ok = false;
                else if (sh >= 0) X = (int64_t)m << sh;
                else if (sh > -24 && (m & ((1u << -sh) - 1u)) == 0) X = (int64_t)(m >> -sh);
                else if (m != 0) ok = false;
                if (bits >> 31) X = -X;
                // offset binary: digit l = byte l of (X + 0x8080808080) - 0x80
                const uint64_t Y = (uint64_t)(X + (int64_t)0x8080808080ll);
                lo[k] = (uint32_t)Y ^ 0x80808080u;
                hi[k] = (uint32_t)(Y >> 32) ^ 0x80u;
            }
            // 4x4 byte transpose of lo[] (plane l = byte l of each element), then plane 4
            const uint32_t a01 = __builtin_amdgcn_perm(lo[1], lo[0], 0x05010400u);
            const uint32_t a23 = __builtin_amdgcn_perm(lo[3], lo[2], 0x05010400u);
            const uint32_t b01 = __builtin_amdgcn_perm(lo[1], lo[0], 0x07030602u);
            const uint32_t b23 = __builtin_amdgcn_perm(lo[3], lo[2], 0x07030602u);
            // a01 = [e0.b0, e1.b0, e0.b1, e1.b1], b01 = [e0.b2, e1.b2, e0.b3, e1.b3]
            const int at = 4 * chunk_slot(kind, q >> 2, n) + (q & 3);  // dword within a plane
            limb[0 * n4 + at] = __builtin_amdgcn_perm(a23, a01, 0x05040100u);
            limb[1 * n4 + at] = __builtin_amdgcn_perm(a23, a01, 0x07060302u);
            limb[2 * n4 + at] = __builtin_amdgcn_perm(b23, b01, 0x05040100u);
            limb[3 * n4 + at] = __builtin_amdgcn_perm(b23, b01, 0x07060302u);
            const uint32_t h01 = __builtin_amdgcn_perm(hi[1], hi[0], 0x0C0C0400u);
            const uint32_t h23 = __builtin_amdgcn_perm(hi[3], hi[2], 0x0C0C0400u);
            limb[4 * n4 + at] = __builtin_amdgcn_perm(h23, h01, 0x05040100u);
            const bool all_ok = uq_group_max<8>(ok ? 0.0f : 1.0f) == 0.0f;
            if ((q & 7) == 0) bexp[q >> 3] = all_ok ? E : -1;
        }
    }
}

// ---- per-kind unit readers
// A lane owns units u = sub, sub + LPR, ... of a row; dot() returns the unit's
// sum over scale groups of scale * sum(code * x).

// 4 IQ4 codes of the low nibbles of the 4 bytes of `nib` (upper nibbles
// ignored), packed as signed bytes: v_perm_b32 over each half of the code
// book, then a third v_perm_b32 takes byte k from the half picked by bit 3 of
// nibble k (selector k, or k + 4 for the upper half).
__device__ __forceinline__ uint32_t iq4_lookup4(uint32_t nib, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
    const uint32_t sel = nib & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel), hi = __builtin_amdgcn_perm(t3, t2, sel);
    const uint32_t pick = ((nib >> 1) & 0x04040404u) | 0x03020100u;
    return __builtin_amdgcn_perm(hi, lo, pick);
}
struct Iq4Book {
    uint32_t t0, t1, t2, t3;
    __device__ Iq4Book() {
        const uint32_t* b = (const uint32_t*)c_iq4;
        t0 = b[0];
        t1 = b[1];
        t2 = b[2];
        t3 = b[3];
    }
};
// the 32 codes of one 16-byte IQ4 unit (low nibbles -> elements 0..15, high -> 16..31)
__device__ __forceinline__ double iq4_dot32(const uint4& w, const XStage& xs, int u, const Iq4Book& bk) {
    const uint32_t v[4] = {w.x, w.y, w.z, w.w};
    uint32_t c[8];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        c[q] = iq4_lookup4(v[q], bk.t0, bk.t1, bk.t2, bk.t3);
        c[4 + q] = iq4_lookup4(v[q] >> 4, bk.t0, bk.t1, bk.t2, bk.t3);
    }
    return seg_dot<2>(c, xs, 32 * u, u, xs.n4 / 8);
}

template <uint32_t K>
struct FK;

// F32 / BF16 weights are not small-integer codes: products in double from x.
template <>
struct FK<KIND_F32> {
    static constexpr int WPU = 8, LPR = 64, CH = 4;
    struct U {
        uint4 a, b;
    };
    static __device__ U load(const FJob& j, int64_t row, int u) {
        const uint4* p = (const uint4*)(j.body + row * j.pitch) + 2 * u;
        return {p[0], p[1]};
    }
    static __device__ double dot(const U& v, const XStage& xs, int u, const uint32_t*, const Iq4Book&) {
        const float* x = xs.xf + 8 * u;
        const float4 xa = ((const float4*)x)[0], xb = ((const float4*)x)[1];
        const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        const uint32_t w[8] = {v.a.x, v.a.y, v.a.z, v.a.w, v.b.x, v.b.y, v.b.z, v.b.w};
        double s[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int k = 0; k < 8; k++) s[k & 3] = __builtin_fma((double)uq_bits_f(w[k]), (double)xv[k], s[k & 3]);
        return (s[0] + s[1]) + (s[2] + s[3]);
    }
};

template <>
struct FK<KIND_BF16> {
    static constexpr int WPU = 8, LPR = 64, CH = 4;
    struct U {
        uint4 a;
    };
    static __device__ U load(const FJob& j, int64_t row, int u) {
        return {((const uint4*)(j.body + row * j.pitch))[u]};
    }
    static __device__ double dot(const U& v, const XStage& xs, int u, const uint32_t*, const Iq4Book&) {
        const float* x = xs.xf + 8 * u;
        const float4 xa = ((const float4*)x)[0], xb = ((const float4*)x)[1];
        const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        const uint32_t w[4] = {v.a.x, v.a.y, v.a.z, v.a.w};
        double s[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            s[k] = __builtin_fma((double)uq_bits_f(w[k] << 16), (double)xv[2 * k], s[k]);
            s[k] = __builtin_fma((double)uq_bits_f(w[k] & 0xFFFF0000u), (double)xv[2 * k + 1], s[k]);
        }
        return (s[0] + s[1]) + (s[2] + s[3]);
    }
};

template <>
struct FK<KIND_Q8_0> {
    static constexpr int WPU = 32, LPR = 16, CH = 4;
    struct U {
        uint4 a, b;
        uint32_t d;
    };
    static __device__ U load(const FJob& j, int64_t row, int u) {
        const uint4* p = (const uint4*)(j.body + row * j.pitch) + 2 * u;
        return {p[0], p[1], j.d[row * (j.n / 32) + u]};
    }
    static __device__ double dot(const U& v, const XStage& xs, int u, const uint32_t*, const Iq4Book&) {
        const uint32_t c[8] = {v.a.x, v.a.y, v.a.z, v.a.w, v.b.x, v.b.y, v.b.z, v.b.w};
        return (double)uq_half((uint16_t)v.d) * seg_dot<2>(c, xs, 32 * u, u, xs.n4 / 8);
    }
};

template <>
struct FK<KIND_IQ4_NL> {
    static constexpr int WPU = 32, LPR = 16, CH = 4;
    struct U {
        uint4 a;
        uint32_t d;
    };
    static __device__ U load(const FJob& j, int64_t row, int u) {
        return {((const uint4*)(j.body + row * j.pitch))[u], j.d[row * (j.n / 32) + u]};
    }
    static __device__ double dot(const U& v, const XStage& xs, int u, const uint32_t*, const Iq4Book& bk) {
        return (double)uq_half((uint16_t)v.d) * iq4_dot32(v.a, xs, u, bk);
    }
};

template <>
struct FK<KIND_IQ4_XS> {
    static constexpr int WPU = 32, LPR = 16, CH = 4;
    struct U {
        uint4 a;
        uint2 h;  // block head: d | scales_h << 16, scales_l
    };
    static __device__ U load(const FJob& j, int64_t row, int u) {
        const uint2 h = ((const uint2*)j.aux)[row * (j.n / 256) + u / 8];
        return {((const uint4*)(j.body + row * j.pitch))[u], h};
    }
    static __device__ double dot(const U& v, const XStage& xs, int u, const uint32_t*, const Iq4Book& bk) {
        const int sb = u & 7;
        const int sc = (int)((v.h.y >> (4 * sb)) & 15) | (int)(((v.h.x >> (16 + 2 * sb)) & 3) << 4);
        const float scale = uq_half((uint16_t)(v.h.x & 0xFFFF)) * (float)(sc - 32);
        return (double)scale * iq4_dot32(v.a, xs, u, bk);
    }
};

// Q6_K unit k = 2*sub + h of a superblock: ql[sub*64 + 16h ..], ql[sub*64 + 32 + 16h ..],
// qh[sub*32 + 16h ..] (16 bytes each) and the 4 group scales sc[sub*8 + h + 2g].
template <>
struct FK<KIND_Q6_K> {
    static constexpr int WPU = 64, LPR = 8, CH = 2;
    struct U {
        uint4 l0, l1, h;
        uint32_t sc, d;
    };
    static __device__ U load(const FJob& j, int64_t row, int u) {
        const uint4* p = (const uint4*)(j.body + row * j.pitch) + 3 * u;
        const uint32_t sc = ((const uint32_t*)j.aux)[row * (j.n / 64) + u];
        return {p[0], p[1], p[2], sc, j.d[row * (j.n / 256) + u / 4]};
    }
    static __device__ double dot(const U& v, const XStage& xs, int u, const uint32_t*, const Iq4Book&) {
        const int e0 = 256 * (u >> 2) + 128 * ((u >> 1) & 1) + 16 * (u & 1);
        const float d = uq_half((uint16_t)v.d);
        const uint32_t l0[4] = {v.l0.x, v.l0.y, v.l0.z, v.l0.w}, l1[4] = {v.l1.x, v.l1.y, v.l1.z, v.l1.w};
        const uint32_t hh[4] = {v.h.x, v.h.y, v.h.z, v.h.w};
        double r = 0.0;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t c[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t lo = ((g & 1 ? l1[q] : l0[q]) >> (4 * (g >> 1))) & 0x0F0F0F0Fu;
                // 6-bit code with bit 5 flipped, its sign bit copied to bits 6-7: code - 32
                const uint32_t t = (lo | (((hh[q] >> (2 * g)) & 0x03030303u) << 4)) ^ 0x20202020u;
                const uint32_t s5 = t & 0x20202020u;
                c[q] = t | (s5 << 1) | (s5 << 2);
            }
            const float scale = d * (float)(int8_t)(uint8_t)(v.sc >> (8 * g));
            r = __builtin_fma((double)scale, seg_dot<1>(c, xs, e0 + 32 * g, g * (xs.n4 / 16) + u, 0), r);
        }
        return r;
    }
};

// IQ3_XXS unit k of a superblock: grid indices of sub-blocks 4k..4k+3 (32
// bytes) then their 4 sign/scale words (16 bytes).
template <>
struct FK<KIND_IQ3_XXS> {
    static constexpr int WPU = 128, LPR = 8, CH = 2;
    struct U {
        uint4 q0, q1, a;
        uint32_t d;
    };
    static __device__ U load(const FJob& j, int64_t row, int u) {
        const uint4* p = (const uint4*)(j.body + row * j.pitch) + 3 * u;
        return {p[0], p[1], p[2], j.d[row * (j.n / 256) + u / 2]};
    }
    // grid bytes (<= 62) negated where the sign mask byte is 0xFF: (g ^ m) + (m & 1),
    // with no carry between bytes
    static __device__ double dot(const U& v, const XStage& xs, int u, const uint32_t* grid, const Iq4Book&) {
        const float d = uq_half((uint16_t)v.d);
        const uint32_t qs[8] = {v.q0.x, v.q0.y, v.q0.z, v.q0.w, v.q1.x, v.q1.y, v.q1.z, v.q1.w};
        const uint32_t aux[4] = {v.a.x, v.a.y, v.a.z, v.a.w};
        double r = 0.0;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            uint32_t c[8];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint4 sm = ((const uint4*)(grid + 256))[(aux[l] >> (7 * g)) & 127u];
                const uint32_t word = qs[2 * l + (g >> 1)];
                const uint32_t g0 = grid[(word >> (16 * (g & 1))) & 255], g1 = grid[(word >> (16 * (g & 1) + 8)) & 255];
                c[2 * g] = (g0 ^ sm.x) + sm.z;
                c[2 * g + 1] = (g1 ^ sm.y) + sm.w;
            }
            const float scale = d * (0.5f + (float)(aux[l] >> 28)) * 0.5f;
            r = __builtin_fma((double)scale, seg_dot<2>(c, xs, 128 * u + 32 * l, 2 * l * (xs.n4 / 32) + u, xs.n4 / 32), r);
        }
        return r;
    }
};

// Rows of one job for workgroup `wgi` of `wgc`: LPR lanes per row, 64/LPR
// rows per wave, row blocks wgi, wgi + wgc, ... A lane owns units u = sub +
// LPR*i of its row and walks them in chunks of CH units: the next chunk's
// loads (the same row's or the next row block's) are issued before the
// current chunk's dots. Per row the lane adds its units in order; the lane
// group sums in double and rounds once.
template <class T>
__device__ void job_rows(const FJob& j, int wgi, int wgc, const XStage& xs, const uint32_t* grid) {
    constexpr int LPR = T::LPR, CH = T::CH, RPW = 64 / LPR;
    const int RPB = RPW * (int)(blockDim.x / 64);  // rows per row block: the launch picks 256 or 512 threads
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane % LPR, grp = lane / LPR;
    const int nu = j.n / T::WPU;
    const int nb = (nu + LPR - 1) / LPR;    // unit slots per lane and row
    const int nch = (nb + CH - 1) / CH;      // chunks per row
    const int64_t rblocks = (j.m + RPB - 1) / RPB;
    if (wgi >= rblocks) return;
    const Iq4Book bk;
    typename T::U buf[2][CH];
    // (row block, chunk) of the next fetch, advanced without division
    int64_t frb = wgi;
    int fc = 0;
    auto fetch = [&](typename T::U (&b)[CH]) {
        const int64_t row = frb * RPB + wave * RPW + grp;
        const int64_t rr = row < j.m ? row : j.m - 1;
#pragma unroll
        for (int k = 0; k < CH; k++) {
            const int u = sub + LPR * (fc * CH + k);
            if (fc * CH + k < nb) b[k] = T::load(j, rr, u < nu ? u : nu - 1);  // slot test is wave-uniform
        }
        if (++fc == nch) {
            fc = 0;
            frb += wgc;
        }
    };
    fetch(buf[0]);
    int64_t rb = wgi;
    int c = 0;
    double acc = 0.0;
    while (rb < rblocks) {
        // two chunks per trip so the chunk buffers keep fixed registers
#pragma unroll
        for (int h = 0; h < 2; h++) {
            if (rb < rblocks) {
                if (frb < rblocks) fetch(buf[h ^ 1]);
#pragma unroll
                for (int k = 0; k < CH; k++) {
                    const int u = sub + LPR * (c * CH + k);
                    if (c * CH + k < nb) {
                        const double d = T::dot(buf[h][k], xs, u < nu ? u : nu - 1, grid, bk);
                        acc = acc + (u < nu ? d : 0.0);
                    }
                }
                if (++c == nch) {
                    const int64_t row = rb * RPB + wave * RPW + grp;
                    const double sum = uq_group_sum<LPR>(acc);
                    if (row < j.m && sub == 0) j.y[row] = (float)sum;
                    acc = 0.0;
                    c = 0;
                    rb += wgc;
                }
            }
        }
    }
}

template <class T>
constexpr int rows_per_wave() {
    return 64 / T::LPR;
}

// Up to MAX_JOBS jobs per launch, passed by value in the kernel arguments
// (no device table to copy before the launch); longer tables take several
// launches, each row computed the same way.
constexpr int MAX_JOBS = 32;
struct JobArgs {
    FJob job[MAX_JOBS];
    int count;
};

// Shared front of the linear kernels: the workgroup's job (wg0 ascending)
// and its staged x.
__device__ __forceinline__ FJob find_job(const JobArgs& a) {
    int lo = 0, hi = a.count;
    while (lo + 1 < hi) {
        const int mid = (lo + hi) >> 1;
        if (a.job[mid].wg0 <= (int)blockIdx.x) lo = mid;
        else hi = mid;
    }
    return a.job[lo];
}
template <bool INTS>
__device__ __forceinline__ XStage stage_job(const FJob& j, uint32_t* fl_lds, uint32_t* lgrid) {
    XStage xs;
    xs.limb = fl_lds;
    xs.bexp = (const int*)(fl_lds + NLIMB * (j.n / 4));
    xs.xg = j.x;
    xs.xf = (const float*)fl_lds;
    xs.n4 = j.n / 4;
    if (INTS) stage_x(j.x, j.n, (uint32_t)j.kind, fl_lds, (int*)(fl_lds + NLIMB * (j.n / 4)));
    else
        for (int i = threadIdx.x; i < j.n / 4; i += (int)blockDim.x) ((float4*)fl_lds)[i] = ((const float4*)j.x)[i];
    for (int i = threadIdx.x; i < 256; i += (int)blockDim.x) lgrid[i] = c_iq3_grid[i];
    // IQ3_XXS signs after the grid: entry s7 (7 stored sign bits, the 8th their
    // parity) = byte masks of values 0-3 and 4-7 (0xFF = negative) and the
    // masks' low bits
    for (int i = threadIdx.x; i < 128; i += (int)blockDim.x) {
        const uint32_t sg = (uint32_t)i | ((uint32_t)(__popc(i) & 1) << 7);
        uint32_t m[2];
        for (int h = 0; h < 2; h++) {
            uint32_t v = 0;
            for (int k = 0; k < 4; k++)
                if ((sg >> (4 * h + k)) & 1) v |= 0xFFu << (8 * k);
            m[h] = v;
        }
        ((uint4*)(lgrid + 256))[i] = make_uint4(m[0], m[1], m[0] & 0x01010101u, m[1] & 0x01010101u);
    }
    __syncthreads();
    return xs;
}

// Jobs of one kind: registers sized for that kind alone.
template <uint32_t K>
__global__ __launch_bounds__(FL_WG) void k_flinear_kind(JobArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint32_t fl_lds[];
    __shared__ __attribute__((aligned(16))) uint32_t lgrid[256 + 4 * 128];  // IQ3 grid, then the sign table
    const FJob j = find_job(a);
    const XStage xs = stage_job<K != KIND_F32 && K != KIND_BF16>(j, fl_lds, lgrid);
    job_rows<FK<K>>(j, (int)blockIdx.x - j.wg0, j.wgs, xs, lgrid);
}

// One launch over a job table of mixed kinds (wg0 ascending): the workgroup finds its job,
// stages that job's x (integer digit planes and block exponents) and the IQ3
// grid in LDS, and runs its rows. Dynamic LDS: NLIMB * n + 4 * (n / 32) bytes
// (F32 / BF16 weights: x as 4 * n bytes of f32).
__global__ __launch_bounds__(FL_WG) void k_flinear(JobArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint32_t fl_lds[];
    __shared__ __attribute__((aligned(16))) uint32_t lgrid[256 + 4 * 128];  // IQ3 grid, then the sign table
    const FJob j = find_job(a);
    const int wgi = (int)blockIdx.x - j.wg0, wgc = j.wgs;
    if (j.kind == KIND_F32 || j.kind == KIND_BF16) {
        const XStage xs = stage_job<false>(j, fl_lds, lgrid);
        if (j.kind == KIND_F32) job_rows<FK<KIND_F32>>(j, wgi, wgc, xs, lgrid);
        else job_rows<FK<KIND_BF16>>(j, wgi, wgc, xs, lgrid);
        return;
    }
    const XStage xs = stage_job<true>(j, fl_lds, lgrid);
    switch (j.kind) {
    case KIND_Q8_0: job_rows<FK<KIND_Q8_0>>(j, wgi, wgc, xs, lgrid); break;
    case KIND_IQ4_NL: job_rows<FK<KIND_IQ4_NL>>(j, wgi, wgc, xs, lgrid); break;
    case KIND_IQ4_XS: job_rows<FK<KIND_IQ4_XS>>(j, wgi, wgc, xs, lgrid); break;
    case KIND_Q6_K: job_rows<FK<KIND_Q6_K>>(j, wgi, wgc, xs, lgrid); break;
    case KIND_IQ3_XXS: job_rows<FK<KIND_IQ3_XXS>>(j, wgi, wgc, xs, lgrid); break;
    default: break;
    }
}

// The kernel for a job table: the kind's own kernel when every job has that kind.
using FlKernel = void (*)(JobArgs);
FlKernel kernel_for(const JobArgs& a) {
    const int32_t k = a.job[0].kind;
    for (int i = 1; i < a.count; i++)
        if (a.job[i].kind != k) return k_flinear;
    switch (k) {
    case KIND_F32: return k_flinear_kind<KIND_F32>;
    case KIND_BF16: return k_flinear_kind<KIND_BF16>;
    case KIND_Q8_0: return k_flinear_kind<KIND_Q8_0>;
    case KIND_IQ4_NL: return k_flinear_kind<KIND_IQ4_NL>;
    case KIND_IQ4_XS: return k_flinear_kind<KIND_IQ4_XS>;
    case KIND_Q6_K: return k_flinear_kind<KIND_Q6_K>;
    case KIND_IQ3_XXS: return k_flinear_kind<KIND_IQ3_XXS>;
    }
    return k_flinear;
}

// Workgroups of a linear kernel resident per CU at `lds` dynamic bytes
// (occupancy query, cached per kernel and size).
int fl_resident(const void* kern, size_t lds) {
    struct Entry {
        const void* k;
        size_t lds;
        int n;
    };
    static Entry cache[64];
    static int used = 0;
    for (int i = 0; i < used; i++)
        if (cache[i].k == kern && cache[i].lds == lds) return cache[i].n;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, FL_WG, lds) != hipSuccess || n <= 0) n = 1;
    if (n > 8) n = 8;
    if (used < 64) cache[used++] = Entry{kern, lds, n};
    return n;
}

size_t stage_bytes(uint32_t kind, int n) {
    return (kind == KIND_F32 || kind == KIND_BF16) ? 4 * (size_t)n : (size_t)NLIMB * n + 4 * (size_t)(n / 32);
}

int wave_rows(uint32_t kind) {
    switch (kind) {
    case KIND_F32: return rows_per_wave<FK<KIND_F32>>();
    case KIND_BF16: return rows_per_wave<FK<KIND_BF16>>();
    case KIND_Q8_0: return rows_per_wave<FK<KIND_Q8_0>>();
    case KIND_IQ4_NL: return rows_per_wave<FK<KIND_IQ4_NL>>();
    case KIND_IQ4_XS: return rows_per_wave<FK<KIND_IQ4_XS>>();
    case KIND_Q6_K: return rows_per_wave<FK<KIND_Q6_K>>();
    case KIND_IQ3_XXS: return rows_per_wave<FK<KIND_IQ3_XXS>>();
    }
    return 0;
}

bool linear_kind(uint32_t kind) { return wave_rows(kind) > 0; }

}  // namespace

// Plane layout of an uploaded frontier kind (the Q8_0 split is the matvec's:
// int8 plane + fp16 plane). Returns false for kinds without one.
bool frontier_layout(uint32_t kind, FrontierLayout& L) {
    std::memset(&L, 0, sizeof(L));
    auto put = [&](int o, int plane, int off) { L.map[o] = (uint16_t)((plane << 12) | off); };
    switch (kind) {
    case KIND_F32:
    case KIND_BF16:
        // 16-byte blocks copied as they are (n % 8 == 0)
        L.block_vals = kind == KIND_F32 ? 4 : 8;
        L.block_bytes = 16;
        L.plane_bytes[0] = 16;
        for (int o = 0; o < 16; o++) put(o, 0, o);
        return true;
    case KIND_IQ4_NL:
        L.block_vals = 32;
        L.block_bytes = 18;
        L.plane_bytes[0] = 16;
        L.plane_bytes[2] = 2;
        put(0, 2, 0);
        put(1, 2, 1);
        for (int o = 2; o < 18; o++) put(o, 0, o - 2);
        return true;
    case KIND_IQ4_XS:
        L.block_vals = 256;
        L.block_bytes = 136;
        L.plane_bytes[0] = 128;
        L.plane_bytes[1] = 8;
        for (int o = 0; o < 8; o++) put(o, 1, o);
        for (int o = 8; o < 136; o++) put(o, 0, o - 8);
        return true;
    case KIND_Q6_K:
        L.block_vals = 256;
        L.block_bytes = 210;
        L.plane_bytes[0] = 192;
        L.plane_bytes[1] = 16;
        L.plane_bytes[2] = 2;
        for (int o = 0; o < 128; o++) {  // ql
            const int sub = o / 64, r = o % 64, half = r / 32, h = (r % 32) / 16, t = r % 16;
            put(o, 0, 48 * (2 * sub + h) + 16 * half + t);
        }
        for (int o = 128; o < 192; o++) {  // qh
            const int r = o - 128, sub = r / 32, h = (r % 32) / 16, t = r % 16;
            put(o, 0, 48 * (2 * sub + h) + 32 + t);
        }
        for (int o = 192; o < 208; o++) {  // scales: byte sub*8 + h + 2g -> unit 2*sub+h, slot g
            const int i = o - 192, sub = i / 8, w = i % 8, h = w % 2, g = w / 2;
            put(o, 1, 4 * (2 * sub + h) + g);
        }
        put(208, 2, 0);
        put(209, 2, 1);
        return true;
    case KIND_IQ3_XXS:
        L.block_vals = 256;
        L.block_bytes = 98;
        L.plane_bytes[0] = 96;
        L.plane_bytes[2] = 2;
        put(0, 2, 0);
        put(1, 2, 1);
        for (int o = 2; o < 66; o++) {  // grid indices
            const int r = o - 2;
            put(o, 0, 48 * (r / 32) + r % 32);
        }
        for (int o = 66; o < 98; o++) {  // sign/scale words
            const int r = o - 66;
            put(o, 0, 48 * (r / 16) + 32 + r % 16);
        }
        return true;
    }
    return false;
}

static MapArgs map_args(const FrontierLayout& L) {
    MapArgs a;
    std::memcpy(a.map, L.map, sizeof(a.map));
    a.block_bytes = L.block_bytes;
    for (int i = 0; i < 3; i++) a.plane_bytes[i] = L.plane_bytes[i];
    return a;
}

static int grid_blocks(int64_t total) {
    const int64_t g = (total + FWG - 1) / FWG;
    return (int)std::min<int64_t>(std::max<int64_t>(g, 1), 65536);
}

void launch_layout_repack(const uint8_t* src, int64_t blocks, const FrontierLayout& L, uint8_t* const planes[3],
                          hipStream_t s) {
    hipLaunchKernelGGL(k_layout_repack, dim3(grid_blocks(blocks * L.block_bytes)), dim3(FWG), 0, s, src, blocks,
                       map_args(L), planes[0], planes[1], planes[2]);
}

void launch_layout_verify(const uint8_t* src, int64_t blocks, const FrontierLayout& L, uint8_t* const planes[3],
                          unsigned* bad, hipStream_t s) {
    hipLaunchKernelGGL(k_layout_verify, dim3(grid_blocks(blocks * L.block_bytes)), dim3(FWG), 0, s, src, blocks,
                       map_args(L), planes[0], planes[1], planes[2], bad);
}

}  // namespace uq

using namespace uq;

namespace {

FJob make_job(const Weight& w, const float* x, float* y) {
    FJob j{};
    j.body = (const uint8_t*)w.qs;
    j.aux = w.sc;
    j.d = w.d;
    j.x = x;
    j.y = y;
    j.m = w.m;
    j.kind = (int32_t)w.kind;
    j.n = (int32_t)w.n;
    switch (w.kind) {
    case KIND_F32: j.pitch = 4 * w.n; break;
    case KIND_BF16: j.pitch = 2 * w.n; break;
    case KIND_Q8_0: j.pitch = w.n; break;
    case KIND_IQ4_NL:
    case KIND_IQ4_XS: j.pitch = w.n / 2; break;
    case KIND_Q6_K: j.pitch = w.n / 256 * 192; break;
    case KIND_IQ3_XXS: j.pitch = w.n / 256 * 96; break;
    }
    return j;
}

int check_job_weight(const uq_weight_t w) {
    if (!w) return set_error(ERR_ARG, "linear: null weight");
    if (!linear_kind(w->w.kind))
        return set_error(ERR_QUANT_TYPE, "linear: the fp32-activation reader takes F32, BF16, Q8_0, Q6_K, IQ3_XXS, "
                                         "IQ4_NL or IQ4_XS weights (frontier_core.rs:53-58)");
    return OK;
}

int enqueue_jobs(const uq_linear_job* jobs, int count, hipStream_t s) {
    if (!jobs || count <= 0) return set_error(ERR_ARG, "linear: empty job table");
    for (int i = 0; i < count; i++) {
        if (int rc = check_job_weight(jobs[i].weight)) return rc;
        if (!jobs[i].x || !jobs[i].y) return set_error(ERR_ARG, "linear: null x or y");
        if ((uintptr_t)jobs[i].x & 15) return set_error(ERR_ARG, "linear: x must be 16-byte aligned");
    }
    for (int c0 = 0; c0 < count; c0 += MAX_JOBS) {
        JobArgs a{};
        a.count = std::min(MAX_JOBS, count - c0);
        size_t lds = 0;
        for (int i = 0; i < a.count; i++) {
            const Weight& w = jobs[c0 + i].weight->w;
            a.job[i] = make_job(w, jobs[c0 + i].x, jobs[c0 + i].y);
            lds = std::max(lds, stage_bytes(w.kind, (int)w.n));
        }
        // each job gets at most as many workgroups as fit on the chip at once
        // (every workgroup loops over its row blocks); a table that cannot fill
        // the chip with 512-thread workgroups runs 256-thread ones, twice as many
        const FlKernel kern = kernel_for(a);
        const int64_t cu = cu_count();
        int threads = FL_WG;
        int64_t wg = 0;
        for (int pass = 0; pass < 2; pass++) {
            const int64_t cap = cu * fl_resident((const void*)kern, lds) * (FL_WG / threads);
            wg = 0;
            for (int i = 0; i < a.count; i++) {
                const Weight& w = jobs[c0 + i].weight->w;
                const int64_t rpb = (int64_t)wave_rows(w.kind) * (threads / 64);
                const int64_t rblocks = (w.m + rpb - 1) / rpb;
                a.job[i].wg0 = (int32_t)wg;
                a.job[i].wgs = (int32_t)std::min<int64_t>(rblocks, cap);
                wg += a.job[i].wgs;
            }
            if (pass == 0 && wg < 2 * cu) threads = FL_WG / 2;
            else break;
        }
        if (wg > 0x7fffffff) return set_error(ERR_SHAPE, "linear: job table too large for one launch");
        static bool lds_set = false;
        if (!lds_set) {
            const FlKernel all[] = {k_flinear, k_flinear_kind<KIND_F32>, k_flinear_kind<KIND_BF16>,
                                    k_flinear_kind<KIND_Q8_0>, k_flinear_kind<KIND_IQ4_NL>,
                                    k_flinear_kind<KIND_IQ4_XS>, k_flinear_kind<KIND_Q6_K>,
                                    k_flinear_kind<KIND_IQ3_XXS>};
            for (FlKernel f : all)
                UQ_CHECK_HIP(hipFuncSetAttribute((const void*)f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)stage_bytes(KIND_Q8_0, 16384)));
            lds_set = true;
        }
        hipLaunchKernelGGL(kern, dim3((unsigned)wg), dim3(threads), lds, s, a);
        UQ_CHECK_HIP(hipGetLastError());
    }
    return OK;
}

int check_finite(const float* v, int64_t n, const char* what) {
    for (int64_t i = 0; i < n; i++)
        if (!std::isfinite(v[i])) return set_error(ERR_NONFINITE, std::string(what) + ": non-finite value");
    return OK;
}

}  // namespace


extern "C" {

int uq_dequantize(uint32_t kind, const void* bytes, size_t nbytes, int64_t n, float* out) {
    if (!uq_stream()) return set_error(ERR_ARG, "uq_init has not been called");
    if (!bytes || !out) return set_error(ERR_ARG, "dequantize: null pointer");
    const int64_t rb = row_bytes(kind, n);
    if (rb == ERR_QUANT_TYPE || kind == KIND_Q3_K || kind == KIND_Q4_K)
        return set_error(ERR_QUANT_TYPE, "dequantize: unsupported kind (frontier_core.rs:53-58)");
    if (rb < 0) return set_error(ERR_SHAPE, "dequantize: n is not a whole number of blocks");
    if ((int64_t)nbytes != rb) return set_error(ERR_SHAPE, "dequantize: byte count != row_bytes(kind, n)");
    hipStream_t s = (hipStream_t)uq_stream();
    const size_t in_bytes = ((size_t)rb + 255) & ~(size_t)255;
    void* stage = nullptr;
    if (int rc = staging_buffer(in_bytes + sizeof(float) * (size_t)n, &stage)) return rc;
    uint8_t* const din = (uint8_t*)stage;
    float* const dout = (float*)((char*)stage + in_bytes);
    hipError_t e = hipMemcpyAsync(din, bytes, (size_t)rb, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(k_dequant, dim3(grid_blocks(n)), dim3(FWG), 0, s, din, dout, kind, n);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpyAsync(out, dout, sizeof(float) * (size_t)n, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return set_error(ERR_DEVICE, std::string("dequantize: ") + hipGetErrorString(e));
    return OK;
}

int uq_linear_multi_dev(const uq_linear_job* jobs, int count, void* stream) {
    if (!uq_stream()) return set_error(ERR_ARG, "uq_init has not been called");
    return enqueue_jobs(jobs, count, stream ? (hipStream_t)stream : (hipStream_t)uq_stream());
}

int uq_linear_dev(uq_weight_t w, const float* x, float* y, void* stream) {
    const uq_linear_job j{w, x, y};
    return uq_linear_multi_dev(&j, 1, stream);
}

int uq_linear_batch(const uq_linear_job* jobs, int count) {
    if (!uq_stream()) return set_error(ERR_ARG, "uq_init has not been called");
    if (!jobs || count <= 0) return set_error(ERR_ARG, "linear_batch: empty job table");
    int64_t xs = 0, ys = 0;
    for (int i = 0; i < count; i++) {
        if (int rc = check_job_weight(jobs[i].weight)) return rc;
        if (!jobs[i].x || !jobs[i].y) return set_error(ERR_ARG, "linear_batch: null x or y");
        xs += jobs[i].weight->w.n;
        ys += jobs[i].weight->w.m;
    }
    for (int i = 0; i < count; i++)
        if (int rc = check_finite(jobs[i].x, jobs[i].weight->w.n, "linear_batch: input")) return rc;
    hipStream_t s = (hipStream_t)uq_stream();
    const size_t x_bytes = (sizeof(float) * (size_t)xs + 255) & ~(size_t)255;
    void* stage = nullptr;
    if (int rc = staging_buffer(x_bytes + sizeof(float) * (size_t)ys, &stage)) return rc;
    float* const dx = (float*)stage;
    float* const dy = (float*)((char*)stage + x_bytes);
    hipError_t e = hipSuccess;
    int rc = OK;
    std::vector<uq_linear_job> dj((size_t)count);
    std::vector<float> host((size_t)ys);
    int64_t xo = 0, yo = 0;
    for (int i = 0; i < count && e == hipSuccess; i++) {
        const Weight& w = jobs[i].weight->w;
        e = hipMemcpyAsync(dx + xo, jobs[i].x, sizeof(float) * (size_t)w.n, hipMemcpyHostToDevice, s);
        dj[(size_t)i] = uq_linear_job{jobs[i].weight, dx + xo, dy + yo};
        xo += w.n;  // n % 8 == 0 keeps every x 32-byte aligned
        yo += w.m;
    }
    if (e == hipSuccess) rc = enqueue_jobs(dj.data(), count, s);
    if (e == hipSuccess && rc == OK)
        e = hipMemcpyAsync(host.data(), dy, sizeof(float) * (size_t)ys, hipMemcpyDeviceToHost, s);
    // a failed enqueue still leaves the copies above reading the staging buffer
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return set_error(ERR_DEVICE, std::string("linear_batch: ") + hipGetErrorString(e));
    if (rc != OK) return rc;
    yo = 0;
    for (int i = 0; i < count; i++) {
        const int64_t m = jobs[i].weight->w.m;
        std::memcpy(jobs[i].y, host.data() + yo, sizeof(float) * (size_t)m);
        yo += m;
    }
    return check_finite(host.data(), ys, "linear_batch: output");
}

int uq_time_linear(const uq_weight_t* ws, int count, int reps, int warmup, double* total_ms) {
    if (!uq_stream()) return set_error(ERR_ARG, "uq_init has not been called");
    if (!ws || count <= 0 || reps <= 0 || warmup < 0 || !total_ms) return set_error(ERR_ARG, "time_linear: bad args");
    int64_t xs = 0, ys = 0;
    for (int i = 0; i < count; i++) {
        if (int rc = check_job_weight(ws[i])) return rc;
        xs += ws[i]->w.n;
        ys += ws[i]->w.m;
    }
    hipStream_t s = (hipStream_t)uq_stream();
    float *dx = nullptr, *dy = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    UQ_CHECK_HIP(hipMalloc(&dx, sizeof(float) * (size_t)xs));
    hipError_t e = hipMalloc(&dy, sizeof(float) * (size_t)ys);
    if (e == hipSuccess) e = hipMemsetAsync(dx, 0, sizeof(float) * (size_t)xs, s);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    int rc = OK;
    std::vector<uq_linear_job> jobs((size_t)count);
    int64_t xo = 0, yo = 0;
    for (int i = 0; i < count; i++) {
        jobs[(size_t)i] = uq_linear_job{ws[i], dx + xo, dy + yo};
        xo += ws[i]->w.n;
        yo += ws[i]->w.m;
    }
    for (int r = 0; r < warmup + reps && e == hipSuccess && rc == OK; r++) {
        if (r == warmup) e = hipEventRecord(e0, s);
        for (int i = 0; i < count && rc == OK; i++) rc = enqueue_jobs(&jobs[(size_t)i], 1, s);
    }
    if (e == hipSuccess && rc == OK) e = hipEventRecord(e1, s);
    if (e == hipSuccess && rc == OK) e = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (e == hipSuccess && rc == OK) e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamSynchronize(s);
    (void)hipFree(dx);
    if (dy) (void)hipFree(dy);
    if (e != hipSuccess) return set_error(ERR_DEVICE, std::string("time_linear: ") + hipGetErrorString(e));
    if (rc != OK) return rc;
    *total_ms = ms;
    return OK;
}

int uq_time_linear_tables(const uq_linear_job* jobs, const int* sizes, int ntables, int reps, double* total_ms) {
    if (!uq_stream()) return set_error(ERR_ARG, "uq_init has not been called");
    if (!jobs || !sizes || ntables <= 0 || reps <= 0 || !total_ms) return set_error(ERR_ARG, "time_linear_tables: bad args");
    hipStream_t s = (hipStream_t)uq_stream();
    hipEvent_t e0 = nullptr, e1 = nullptr;
    UQ_CHECK_HIP(hipEventCreate(&e0));
    hipError_t e = hipEventCreate(&e1);
    int rc = OK;
    for (int r = 0; r <= reps && e == hipSuccess && rc == OK; r++) {  // round 0 untimed
        if (r == 1) e = hipEventRecord(e0, s);
        int off = 0;
        for (int t = 0; t < ntables && rc == OK; t++) {
            rc = enqueue_jobs(jobs + off, sizes[t], s);
            off += sizes[t];
        }
    }
    if (e == hipSuccess && rc == OK) e = hipEventRecord(e1, s);
    if (e == hipSuccess && rc == OK) e = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (e == hipSuccess && rc == OK) e = hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (e != hipSuccess) return set_error(ERR_DEVICE, std::string("time_linear_tables: ") + hipGetErrorString(e));
    if (rc != OK) return rc;
    *total_ms = ms;
    return OK;
}

int uq_linear(uq_weight_t w, const float* x, int64_t n, float* y, int64_t m) {
    if (!w) return set_error(ERR_ARG, "linear: null weight");
    if (w->w.n != n || w->w.m != m) return set_error(ERR_SHAPE, "linear: tensor shape != x/y lengths");
    const uq_linear_job j{w, x, y};
    return uq_linear_batch(&j, 1);
}

}  // extern "C"
