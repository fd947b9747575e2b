// Device-side arithmetic shared by every gfx950 kernel of the path.
//
// Numeric contract (the same one the CPU oracle follows):
//  * all HIP code is built with -ffp-contract=off; f32 elementwise formulas are
//    written op by op in the reference's order;
//  * reductions accumulate exactly formed double terms and round to f32 once,
//    so the result does not depend on the lane/wave summation order;
//  * exp is uq_expf below (double Cody-Waite + degree-12 Taylor, one rounding),
//    bit-identical to the oracle's restatement.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define UQ_DEV __device__ __forceinline__

UQ_DEV float uq_half(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
UQ_DEV uint16_t uq_f16_rne(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

UQ_DEV float uq_expf(float x) {
    if (x != x) return x;
    if (x > 100.0f) return __builtin_inff();
    if (x < -110.0f) return 0.0f;
    const double xd = (double)x;
    const double kd = __builtin_rint(xd * 0x1.71547652b82fep+0);
    double r = __builtin_fma(-kd, 0x1.62e42fefa39efp-1, xd);
    r = __builtin_fma(-kd, 0x1.abc9e3b39803fp-56, r);
    double p = 0x1.1eed8eff8d898p-29;
    p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);
    p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);
    p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);
    p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);
    p = __builtin_fma(p, r, 0x1.1111111111111p-7);
    p = __builtin_fma(p, r, 0x1.5555555555555p-5);
    p = __builtin_fma(p, r, 0x1.5555555555555p-3);
    p = __builtin_fma(p, r, 0x1.0000000000000p-1);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return (float)__builtin_ldexp(p, (int)kd);
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

UQ_DEV double uq_shfl_xor_d(double v, int mask) {
    int2 p = __builtin_bit_cast(int2, v);
    p.x = __shfl_xor(p.x, mask, 64);
    p.y = __shfl_xor(p.y, mask, 64);
    return __builtin_bit_cast(double, p);
}

// Sum of a double over groups of G consecutive lanes (G a power of two <= 64);
// every lane of the group receives the total.
template <int G>
UQ_DEV double uq_group_sum(double v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v += uq_shfl_xor_d(v, off);
    return v;
}
template <int G>
UQ_DEV float uq_group_max(float v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
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
