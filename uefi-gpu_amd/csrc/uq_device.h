// Device-side arithmetic shared by every gfx950 kernel of the path.
//
// Numeric contract (the same one the CPU oracle follows):
//  * all HIP code is built with -ffp-contract=off; f32 elementwise formulas are
//    written op by op in the reference's order;
//  * reductions accumulate exactly formed double terms and round to f32 once,
//    so the result does not depend on the lane/wave summation order;
//  * exp is uq_expf below, the reference Rust path's libm expf in f32,
//    bit-identical to the oracle's restatement.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define UQ_DEV __device__ __forceinline__
// Also built for the host: the exhaustive check of uq_expf runs there.
#define UQ_HD __host__ __device__ __forceinline__

// s_waitcnt vmcnt(0): every vector-memory op this wave has issued (LDS DMA
// included) has completed; expcnt and lgkmcnt are not waited on.
UQ_DEV void uq_wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// Scalar read (s_load_dword, lgkmcnt) of a value that no thread of the running
// kernel writes; the scalar cache starts every dispatch invalidated. Keeps such
// reads out of the vector-memory counter, so they never wait behind (or hold
// up) the weight stream.
UQ_DEV int uq_sload(const int* p) { return *(const __attribute__((address_space(4))) int*)p; }
// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4):
// lane l's bytes land at lds_wave_base + 16*l; lds_wave_base is wave-uniform.
typedef __attribute__((address_space(3))) void uq_lds_void;
UQ_DEV void uq_lds_load16(const void* g, void* lds_wave_base) {
    __builtin_amdgcn_global_load_lds(g, (uq_lds_void*)lds_wave_base, 16, 0, 0);
}
// Workgroup barrier that waits for no memory operation (s_barrier alone):
// orders instruction issue across the waves, publishes nothing.
UQ_DEV void uq_issue_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}
// a * b for |a|, |b| < 2^23 whose product fits in 32 bits (v_mul_i32_i24, full rate)
UQ_DEV int uq_mul24(int a, int b) { return __mul24(a, b); }
UQ_DEV float uq_half(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
UQ_DEV uint16_t uq_f16_rne(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

UQ_HD float uq_bits_f(uint32_t u) { return __builtin_bit_cast(float, u); }

// expf of the reference's Rust path: libm 0.2.16 (FreeBSD e_expf.c), as
// restated at driver/src/frontier_cpu_expf.rs:80-170. Same f32 operations as
// the oracle's uqo_expf; division is IEEE (HIP's correctly rounded f32 '/').
// Algorithm: Copyright (C) 1993 by Sun Microsystems, Inc.; notice kept in
// third_party/NOTICE.sunpro-expf.
UQ_HD float uq_expf(float x) {
    // Branch-free, and with fewer selects than the branchy form has cases:
    // - k = x/ln2 rounded half away from zero everywhere. The branchy form
    //   takes k = 0 for |x| <= ln2/2 and +-1 up to 1.5 ln2; where the
    //   rounding gives another k there, that reduction yields the same bits.
    // - scalbnf(y, k) as two multiplies by 2^(k>>1) and 2^(k - (k>>1)): the
    //   exact y * 2^k is rounded once either way (only the last multiply can
    //   round, into the subnormal range or to infinity).
    // - the small-|x| result and the special values stay selects.
    // Every one of the 2^32 inputs gives the branchy form's bits (checked
    // exhaustively against the oracle's expf).
    const uint32_t bx = __builtin_bit_cast(uint32_t, x);
    const uint32_t ax = bx & 0x7fffffffu;
    const bool neg = (bx >> 31) != 0;
    const float t = fminf(fmaxf(x * uq_bits_f(0x3fb8aa3bu), -160.0f), 160.0f);
    const int k = (int)(t + (neg ? -0.5f : 0.5f));
    const float kf = (float)k;
    const float hi = x - kf * uq_bits_f(0x3f317200u);
    const float lo = kf * uq_bits_f(0x35bfbe8eu);
    const float xr = hi - lo;
    const float r2 = xr * xr;
    const float poly = r2 * (uq_bits_f(0x3e2aaa8fu) + r2 * uq_bits_f(0xbb355215u));
    const float c = xr - poly;
    const float q = (xr * c) / (2.0f - c);
    const float y = 1.0f + ((q - lo) + hi);
    // |k| <= 161 (t is clamped), so both factors are normal powers of two
    const int ka = k >> 1, kb = k - ka;
    float r = (y * uq_bits_f((uint32_t)(127 + ka) << 23)) * uq_bits_f((uint32_t)(127 + kb) << 23);
    r = ax <= 0x39000000u ? 1.0f + x : r;
    r = neg && ax >= 0x42cff1b5u ? 0.0f : r;
    r = !neg && ax >= 0x42b17218u ? x * 0x1p127f : r;
    return ax > 0x7f800000u ? x : r;
}

// (g / (1 + exp(-g))) * u  -- gateup_dp4a / silu_mul form
UQ_DEV float uq_silu_mul(float g, float u) {
    float e = uq_expf(-g);
    float den = 1.0f + e;
    float s = g / den;
    return s * u;
}
// 1 / (1 + exp(-x))  -- frontier activation(x, false)
UQ_DEV float uq_sigmoid(float x) {
    float e = uq_expf(-x);
    float d = 1.0f + e;
    return 1.0f / d;
}

// 16-byte non-temporal load for weights that are streamed once per launch.
typedef int uq_v4i __attribute__((ext_vector_type(4)));
UQ_DEV int4 uq_ntload16(const void* p) {
    const uq_v4i v = __builtin_nontemporal_load((const uq_v4i*)p);
    return make_int4(v.x, v.y, v.z, v.w);
}
// 12-byte non-temporal load (one global_load_dwordx3), 4-byte aligned.
typedef int uq_v3i __attribute__((ext_vector_type(3), aligned(4)));
UQ_DEV int3 uq_ntload12(const void* p) {
    const uq_v3i v = __builtin_nontemporal_load((const uq_v3i*)p);
    return make_int3(v.x, v.y, v.z);
}

// 4-way signed int8 dot with int32 accumulate (v_dot4_i32_i8).
UQ_DEV int uq_dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

UQ_DEV int uq_dot32(const int4& wa, const int4& wb, const int4& xa, const int4& xb) {
    int c = 0;
    c = uq_dot4(wa.x, xa.x, c); c = uq_dot4(wa.y, xa.y, c);
    c = uq_dot4(wa.z, xa.z, c); c = uq_dot4(wa.w, xa.w, c);
    c = uq_dot4(wb.x, xb.x, c); c = uq_dot4(wb.y, xb.y, c);
    c = uq_dot4(wb.z, xb.z, c); c = uq_dot4(wb.w, xb.w, c);
    return c;
}

// Cross-lane reductions without LDS traffic: DPP lane moves inside rows of 16
// lanes (quad_perm xor 1 and xor 2, row_half_mirror, row_mirror, row_ror:8)
// and the gfx950 permlane16/32 swaps across rows. Every lane of a group ends
// with the same bits (each step adds a value and its partner's, commutatively).
constexpr int UQ_DPP_XOR1 = 0xB1, UQ_DPP_XOR2 = 0x4E, UQ_DPP_MIRROR = 0x140, UQ_DPP_HALF_MIRROR = 0x141,
              UQ_DPP_ROR8 = 0x128;
template <int CTRL>
UQ_DEV int uq_dpp(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false); }
template <int CTRL>
UQ_DEV double uq_dpp_d(double v) {
    int2 p = __builtin_bit_cast(int2, v);
    p.x = uq_dpp<CTRL>(p.x);
    p.y = uq_dpp<CTRL>(p.y);
    return __builtin_bit_cast(double, p);
}
template <int CTRL>
UQ_DEV float uq_dpp_f(float v) { return __builtin_bit_cast(float, uq_dpp<CTRL>(__builtin_bit_cast(int, v))); }
// rows (0,1) and (2,3) of 16 lanes, or halves of 32 lanes, summed / maxed
UQ_DEV double uq_swap16_sum(double v) {
    const int2 p = __builtin_bit_cast(int2, v);
    const auto a = __builtin_amdgcn_permlane16_swap(p.x, p.x, false, false);
    const auto b = __builtin_amdgcn_permlane16_swap(p.y, p.y, false, false);
    return __builtin_bit_cast(double, make_int2(a[0], b[0])) + __builtin_bit_cast(double, make_int2(a[1], b[1]));
}
UQ_DEV double uq_swap32_sum(double v) {
    const int2 p = __builtin_bit_cast(int2, v);
    const auto a = __builtin_amdgcn_permlane32_swap(p.x, p.x, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(p.y, p.y, false, false);
    return __builtin_bit_cast(double, make_int2(a[0], b[0])) + __builtin_bit_cast(double, make_int2(a[1], b[1]));
}
UQ_DEV float uq_swap16_max(float v) {
    const int i = __builtin_bit_cast(int, v);
    const auto a = __builtin_amdgcn_permlane16_swap(i, i, false, false);
    return fmaxf(__builtin_bit_cast(float, (int)a[0]), __builtin_bit_cast(float, (int)a[1]));
}
UQ_DEV float uq_swap32_max(float v) {
    const int i = __builtin_bit_cast(int, v);
    const auto a = __builtin_amdgcn_permlane32_swap(i, i, false, false);
    return fmaxf(__builtin_bit_cast(float, (int)a[0]), __builtin_bit_cast(float, (int)a[1]));
}

// Sum of a double over groups of G consecutive lanes (G a power of two <= 64);
// every lane of the group receives the total.
template <int G>
UQ_DEV double uq_group_sum(double v) {
    if (G >= 2) v = v + uq_dpp_d<UQ_DPP_XOR1>(v);
    if (G >= 4) v = v + uq_dpp_d<UQ_DPP_XOR2>(v);
    if (G >= 8) v = v + uq_dpp_d<UQ_DPP_HALF_MIRROR>(v);
    if (G >= 16) v = v + uq_dpp_d<UQ_DPP_MIRROR>(v);
    if (G >= 32) v = uq_swap16_sum(v);
    if (G >= 64) v = uq_swap32_sum(v);
    return v;
}
template <int G>
UQ_DEV float uq_group_max(float v) {
    if (G >= 2) v = fmaxf(v, uq_dpp_f<UQ_DPP_XOR1>(v));
    if (G >= 4) v = fmaxf(v, uq_dpp_f<UQ_DPP_XOR2>(v));
    if (G >= 8) v = fmaxf(v, uq_dpp_f<UQ_DPP_HALF_MIRROR>(v));
    if (G >= 16) v = fmaxf(v, uq_dpp_f<UQ_DPP_MIRROR>(v));
    if (G >= 32) v = uq_swap16_max(v);
    if (G >= 64) v = uq_swap32_max(v);
    return v;
}
// Sum over the lanes of a wave with equal lane % LP (LP in 8, 16, 32, 64).
template <int LP>
UQ_DEV double uq_rows_sum(double v) {
    if (LP <= 8) v = v + uq_dpp_d<UQ_DPP_ROR8>(v);
    if (LP <= 16) v = uq_swap16_sum(v);
    if (LP <= 32) v = uq_swap32_sum(v);
    return v;
}

// Block-32 activation quantization of one value per lane, 32 lanes per block
// (gpu_dp4a.cu:23-31): a = max|x| over the block, inv = a>0 ? 127/a : 0,
// q = rint(x*inv) clamped to +-127 (NaN -> 0), scale = a/127.
UQ_DEV int8_t uq_quant_lane(float v, float* scale_out) {
    float a = uq_group_max<32>(fabsf(v));
    float inv = a > 0.0f ? 127.0f / a : 0.0f;
    float t = v * inv;
    float r = __builtin_rintf(t);
    if (r != r) r = 0.0f;
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    *scale_out = a / 127.0f;
    return (int8_t)(int)r;
}
// The same quant with 4 consecutive values per lane, a 32-block = 8 lanes:
// returns the block scale and packs the 4 int8 codes (lowest value in the low
// byte). The amax is an fmaxf tree like uq_quant_lane's (a NaN is dropped
// unless the whole block is NaN), so both give the same codes and scale.
// The code of one value given its block's 127/amax (0 for an all-zero or
// all-NaN block), as uq_quant_lane computes it.
UQ_DEV uint32_t uq_quant_code(float v, float inv) {
    float r = __builtin_rintf(v * inv);
    if (r != r) r = 0.0f;
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return (uint32_t)(uint8_t)(int8_t)(int)r;
}
// 127/amax and amax/127 of NB blocks, each block spread over a G-lane group
// whose lanes all hold its amax (after uq_group_max<G>). An IEEE division
// sequence holds VCC, so the divisions of one lane run one after another;
// here lane r of a group divides for blocks r, r + G, ... and the group's
// lanes run them side by side. Every lane then takes 127/amax of all NB
// blocks back by ds_bpermute. sc[k] is the scale of block r + k*G (meaningful
// where r + k*G < NB). The same operations as uq_quant4_group8 /
// uq_quant_lane per block, so the same bits.
template <int NB, int G>
UQ_DEV void uq_block_recips(const float (&amax)[NB], float (&inv)[NB], float (&sc)[(NB + G - 1) / G]) {
    constexpr int NK = (NB + G - 1) / G;
    const int lane = threadIdx.x & 63, r = lane & (G - 1), base = lane & ~(G - 1);
    float iv[NK];
#pragma unroll
    for (int k = 0; k < NK; k++) {
        float a = amax[k * G];
#pragma unroll
        for (int j = 1; j < G; j++)
            if (k * G + j < NB) a = r == j ? amax[k * G + j] : a;
        iv[k] = a > 0.0f ? 127.0f / a : 0.0f;
        sc[k] = a / 127.0f;
    }
#pragma unroll
    for (int j = 0; j < NB; j++) inv[j] = __shfl(iv[j / G], base + j % G, 64);
}
UQ_DEV float uq_quant4_group8(const float v[4], uint32_t* packed) {
    float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    a = uq_group_max<8>(a);
    const float inv = a > 0.0f ? 127.0f / a : 0.0f;
    uint32_t p = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) p |= uq_quant_code(v[c], inv) << (8 * c);
    *packed = p;
    return a / 127.0f;
}
