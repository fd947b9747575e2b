/*
 * CPU oracle for the quantized-matmul hot path -- TEST INFRASTRUCTURE ONLY.
 * Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg;
 * the product library (libuq.so) never links or calls it.
 *
 * Restates the reference runtime nodnarbrox/uefi-gpu (Rust no_std + CUDA C).
 * Build: gcc -O3 -ffp-contract=off -fopenmp (oracle/Makefile). Threading only
 * splits independent rows/tokens; it never changes an operation order.
 *
 * Parity pins (tests/test_oracle_*.py):
 *   uqo_half            exhaustive 65536 patterns vs numpy float16 (IEEE)
 *   uqo_f16_rne         vs numpy float32->float16 on specials + 4M samples
 *   uqo_expf            libm 0.2.16 expf algorithm (frontier_cpu_expf.rs:80-170):
 *                       polynomial bits of :182-183, every reduction boundary
 *                       of :189-199 against float64 exp, <1 ulp vs float64
 *                       exp on dense and bit-pattern samples
 *   uqo_quant_act       closed form: zero block, ties-to-even, amax -> +-127,
 *                       |q*scale - x| <= scale/2, vs integer brute force
 *   block dots (Q8_0)   int64 numpy brute force
 *   uqo_matvec (Q8_0)   vs float64 exact sum and vs the literal f32 form of
 *                       gpu_prefill.rs:116 (<=1e-3 rel), vs llm.rs:302-309
 *   Q4_K / Q3_K         formats absent from the reference (frontier_core.rs:
 *                       53-58); pinned against ggml's published block structs
 *                       and dequantize_row_q4_K/_q3_K by byte-literal
 *                       superblocks with their expected values written out,
 *                       hand-worked known-answer blocks, integer path ==
 *                       dequant path, encode/decode round trips of the layouts
 *   dequantize, kinds   hand-worked known-answer blocks per kind (code book
 *   BF16/Q6_K/IQ3_XXS/  and grid entries, sign parity, scale composition and
 *   IQ4_NL/IQ4_XS       f32 multiply order), fp16-scale linearity, the IQ3
 *                       grid's invariants; the grid and code book are data of
 *                       the reference (frontier_tables.rs, frontier_core.rs:67)
 *   uqo_linear          vs float64 numpy dot of uqo_dequantize values, and vs
 *                       the reference's f32 check (frontier_gpu.rs:104-111)
 *                       within its 2e-4 + 2e-5|ref| tolerance
 *   uqo_prefill_gemm    int64 brute force + float64 bound; sequential order
 *   uqo_rmsnorm/rope/attention/greedy  float64 textbook forms, invariants
 *                       (softmax sums to 1, pos 0 identity, norm-preserving
 *                       rotation), np.argmax tie rule
 *   uqo_prefill/decode  prefill(n)+decode == token-by-token consistency checks
 *                       and committed golden ids (tests/golden)
 *   uqo_moe_*           routing vs numpy stable argsort, combine vs float64
 *   RoPE powf/sincosf   parity unpinned vs libm 0.2.16 bits (host glibc used by
 *                       both this oracle and the product library; shared by
 *                       construction, checked against float64 within 2 ulp)
 */
#define _GNU_SOURCE
#include "uq_oracle.h"
#include <math.h>
#include <float.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float f_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t bits_from_f(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

void uqo_set_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n > 0 ? n : 1);
#else
    (void)n;
#endif
}
int uqo_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* driver/src/frontier_core.rs:60-65 (also llm.rs:101-106): fp16 -> f32, with
 * the subnormal branch written as frac * 2^-24. */
float uqo_half(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 31u, frac = h & 1023u;
    if (e == 0) { float v = (float)frac * (1.0f / 16777216.0f); return sign ? -v : v; }
    if (e == 31) return f_from_bits(sign | 0x7f800000u | (frac << 13));
    return f_from_bits(sign | ((e + 112u) << 23) | (frac << 13));
}

/* f32 -> fp16 round-to-nearest-even (the fp16 KV cache; the reference keeps an
 * FP32 cache, driver/kernels/gpu_attention.cu:1, the fp16 cache is the
 * requested variant). */
uint16_t uqo_f16_rne(float f) {
    uint32_t x = bits_from_f(f), sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        float a = f_from_bits(ax) * 16777216.0f; /* exact power-of-two scaling */
        return (uint16_t)(sign | (uint32_t)rintf(a));
    }
    uint32_t e = (ax >> 23) - 112u, mant = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (mant >> 13), rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

/* exp for softmax / SiLU / sigmoid: the expf of the reference's Rust path
 * (libm 0.2.16, derived from FreeBSD e_expf.c), called at llm.rs:365,374 and
 * restated instruction by instruction at frontier_cpu_expf.rs:80-170 (whose
 * tests pin the polynomial bits at :182-183). f32 arithmetic throughout:
 *   k = nearest integer to x/ln2 (|x| > 0.5 ln2; +-1 below 1.5 ln2),
 *   hi = x - k*ln2_hi (exact), lo = k*ln2_lo, r = hi - lo,
 *   c = r - r^2 (P1 + r^2 P2),  y = 1 + (r c / (2 - c) - lo + hi),
 *   result = y * 2^k (scalbnf steps for k outside the normal exponent range).
 * The kernels evaluate the same f32 operations (uq_device.h). Algorithm:
 * Copyright (C) 1993 by Sun Microsystems, Inc.; notice kept in
 * third_party/NOTICE.sunpro-expf. */
static float scalbnf_steps(float y, int k) {
    if (k > 127) {
        y = y * 0x1p127f; k -= 127;
        if (k > 127) { y = y * 0x1p127f; k -= 127; if (k > 127) k = 127; }
    } else if (k < -126) {
        y = y * 0x1p-102f; k += 102;
        if (k < -126) { y = y * 0x1p-102f; k += 102; if (k < -126) k = -126; }
    }
    return y * f_from_bits((uint32_t)(127 + k) << 23);
}

float uqo_expf(float x) {
    const uint32_t ax = bits_from_f(x) & 0x7fffffffu;
    const int neg = (int)(bits_from_f(x) >> 31);
    if (ax >= 0x42aeac50u) {                       /* |x| >= 87.3365 or NaN */
        if (ax > 0x7f800000u) return x;            /* NaN */
        if (!neg && ax >= 0x42b17218u) return x * 0x1p127f;  /* overflow */
        if (neg && ax >= 0x42cff1b5u) return 0.0f; /* x <= -103.972 */
    }
    if (ax <= 0x39000000u) return 1.0f + x;        /* |x| <= 2^-14 */
    float hi = x, lo = 0.0f;
    int k = 0;
    if (ax > 0x3eb17218u) {                        /* |x| > 0.5 ln2 */
        if (ax > 0x3f851592u) {                    /* |x| > 1.5 ln2 */
            const float t = x * f_from_bits(0x3fb8aa3bu);
            k = (int)(t + (neg ? -0.5f : 0.5f));   /* truncation */
        } else {
            k = neg ? -1 : 1;
        }
        const float kf = (float)k;
        hi = x - kf * f_from_bits(0x3f317200u);
        lo = kf * f_from_bits(0x35bfbe8eu);
        x = hi - lo;
    }
    const float r2 = x * x;
    const float poly = r2 * (f_from_bits(0x3e2aaa8fu) + r2 * f_from_bits(0xbb355215u));
    const float c = x - poly;
    const float q = (x * c) / (2.0f - c);
    const float y = 1.0f + ((q - lo) + hi);
    return k == 0 ? y : scalbnf_steps(y, k);
}

/* driver/src/frontier_core.rs:53-58 row sizes, extended with the two K-quant
 * layouts the requested configs add (ggml Q3_K 110 B, Q4_K 144 B per 256). */
int64_t uqo_row_bytes(uint32_t kind, int64_t n) {
    int64_t block, bytes;
    switch (kind) {
    case UQO_F32: block = 1; bytes = 4; break;
    case UQO_Q8_0: block = 32; bytes = 34; break;
    case UQO_Q4_K: block = 256; bytes = 144; break;
    case UQO_Q3_K: block = 256; bytes = 110; break;
    /* the reference's remaining kinds, frontier_core.rs:53-58 */
    case UQO_Q6_K: block = 256; bytes = 210; break;
    case UQO_IQ3_XXS: block = 256; bytes = 98; break;
    case UQO_IQ4_NL: block = 32; bytes = 18; break;
    case UQO_IQ4_XS: block = 256; bytes = 136; break;
    case UQO_BF16: block = 1; bytes = 2; break;
    default: return -1;
    }
    if (n <= 0 || n % block) return -2;
    return n / block * bytes;
}

/* ggml get_scale_min_k4: 6-bit scale/min j of a Q4_K superblock. */
static inline void q4k_scale_min(int j, const uint8_t* q, int* sc, int* m) {
    if (j < 4) { *sc = q[j] & 63; *m = q[j + 4] & 63; }
    else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}
/* ggml Q3_K: 6-bit scale s (0..15) of the 12 packed bytes, before the -32. */
static inline int q3k_scale(int s, const uint8_t* sc) {
    int low = s < 8 ? (sc[s] & 0xF) : (sc[s - 8] >> 4);
    int high = (sc[8 + (s & 3)] >> (2 * (s >> 2))) & 3;
    return low | (high << 4);
}
/* ggml Q3_K signed 3-bit value i (0..255) of a superblock: (qs bits) - 4*!hbit. */
static inline int q3k_value(int i, const uint8_t* blk) {
    const uint8_t *hm = blk, *qs = blk + 32;
    int n = i >> 7, j = (i >> 5) & 3, h = (i >> 4) & 1, l = i & 15;
    int low = (qs[32 * n + 16 * h + l] >> (2 * j)) & 3;
    int hb = (hm[16 * h + l] >> (4 * n + j)) & 1;
    return low - (hb ? 0 : 4);
}
/* ggml Q4_K unsigned 4-bit value i (0..255) of a superblock. */
static inline int q4k_value(int i, const uint8_t* blk) {
    const uint8_t* qs = blk + 16;
    int j = i >> 6, h = (i >> 5) & 1, l = i & 31;
    return (qs[32 * j + l] >> (4 * h)) & 15;
}

/* driver/src/frontier_core.rs:73-106 form (one value at a time, ggml's scale
 * multiplication order), for F32, Q8_0 and the Q4_K/Q3_K layouts. */
/* ggml data (MIT licence, third_party/LICENSE.ggml).
 * The IQ4_NL/IQ4_XS code book (frontier_core.rs:67) and the IQ3_XXS grid
 * (frontier_tables.rs:2-35, ggml's iq3xxs_grid). The grid is held here in a
 * different encoding than the product's: entry i as four 3-bit digits (lowest
 * byte first) into the eight byte levels below, expanded by uqo_iq3_grid();
 * the tests check the expansion's invariants (256 distinct entries in
 * ascending order, every byte one of the levels). */
static const int8_t IQ4_BOOK[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
static const uint8_t IQ3_LEVEL[8] = {4, 12, 20, 28, 36, 44, 52, 62};
static const uint16_t IQ3_DIGITS[256] = {
       0,    2,    4,    9,   11,   15,   16,   18,   25,   34,   59,   61,   65,   67,   72,   74,
      81,   85,   88,   90,   97,  108,  120,  128,  130,  132,  137,  144,  146,  153,  155,  159,
     169,  175,  189,  193,  199,  200,  202,  213,  248,  267,  287,  292,  303,  315,  317,  321,
     327,  346,  362,  413,  436,  456,  460,  462,  483,  497,  513,  515,  520,  522,  529,  531,
     536,  538,  540,  551,  552,  576,  578,  585,  592,  594,  641,  643,  648,  650,  657,  664,
     698,  704,  706,  720,  729,  742,  758,  769,  773,  808,  848,  852,  870,  889,  901,  978,
     992, 1024, 1026, 1033, 1035, 1040, 1042, 1046, 1049, 1058, 1089, 1091, 1093, 1096, 1098, 1105,
    1112, 1139, 1143, 1144, 1152, 1154, 1161, 1167, 1168, 1170, 1183, 1184, 1197, 1217, 1224, 1228,
    1272, 1276, 1309, 1323, 1347, 1367, 1377, 1404, 1473, 1475, 1486, 1509, 1537, 1544, 1546, 1553,
    1555, 1576, 1589, 1594, 1600, 1602, 1616, 1625, 1636, 1638, 1665, 1667, 1672, 1685, 1706, 1722,
    1737, 1755, 1816, 1831, 1850, 1856, 1862, 1874, 1901, 1932, 1950, 1971, 2011, 2032, 2052, 2063,
    2077, 2079, 2091, 2095, 2172, 2192, 2207, 2208, 2224, 2230, 2247, 2277, 2308, 2345, 2356, 2389,
    2403, 2424, 2501, 2504, 2506, 2520, 2570, 2593, 2616, 2624, 2630, 2646, 2669, 2700, 2714, 2746,
    2754, 2795, 2824, 2835, 2839, 2874, 2882, 2905, 2984, 3028, 3042, 3092, 3108, 3110, 3124, 3153,
    3185, 3215, 3252, 3288, 3294, 3364, 3397, 3434, 3483, 3523, 3537, 3587, 3589, 3591, 3592, 3610,
    3626, 3670, 3680, 3722, 3749, 3754, 3776, 3789, 3803, 3824, 3857, 3873, 3904, 3906, 3924, 3992,
};
uint32_t uqo_iq3_grid(int i) {
    uint32_t v = 0, d = IQ3_DIGITS[i & 255];
    for (int k = 0; k < 4; k++) v |= (uint32_t)IQ3_LEVEL[(d >> (3 * k)) & 7] << (8 * k);
    return v;
}
int uqo_iq4_value(int i) { return IQ4_BOOK[i & 15]; }
static inline uint32_t rd32(const uint8_t* p) { return (uint32_t)rd16(p) | ((uint32_t)rd16(p + 2) << 16); }

/* Exact decoded value i of a GGUF byte run: frontier_core.rs:73-106 (GPU twin
 * frontier_quant.cu:12-33), with the same f32 multiplication order. */
static float dequant_one(uint32_t kind, const uint8_t* in, int64_t i) {
    switch (kind) {
    case UQO_BF16: return f_from_bits((uint32_t)rd16(in + 2 * i) << 16);
    case UQO_IQ4_NL: {
        const uint8_t* p = in + (i / 32) * 18;
        int j = (int)(i % 32), q = (p[2 + j % 16] >> (4 * (j / 16))) & 15;
        return uqo_half(rd16(p)) * (float)IQ4_BOOK[q];
    }
    case UQO_IQ4_XS: {
        const uint8_t* p = in + (i / 256) * 136;
        int j = (int)(i % 256), sb = j / 32;
        int sc = ((p[4 + sb / 2] >> (4 * (sb % 2))) & 15) | (((rd16(p + 2) >> (2 * sb)) & 3) << 4);
        int q = (p[8 + sb * 16 + j % 16] >> (4 * ((j % 32) / 16))) & 15;
        return (uqo_half(rd16(p)) * (float)(sc - 32)) * (float)IQ4_BOOK[q];
    }
    case UQO_Q6_K: {
        const uint8_t* p = in + (i / 256) * 210;
        int j = (int)(i % 256), sub = j / 128, l = j % 32, g = (j % 128) / 32;
        int lo = p[sub * 64 + l + (g % 2) * 32], hi = p[128 + sub * 32 + l];
        int q = (((lo >> (4 * (g / 2))) & 15) | (((hi >> (2 * g)) & 3) << 4)) - 32;
        int sc = (int8_t)p[192 + sub * 8 + l / 16 + g * 2];
        return (uqo_half(rd16(p + 208)) * (float)sc) * (float)q;
    }
    case UQO_IQ3_XXS: {
        const uint8_t* p = in + (i / 256) * 98;
        int j = (int)(i % 256), sb = j / 32, g = (j % 32) / 8;
        uint32_t aux = rd32(p + 66 + sb * 4), s7 = (aux >> (7 * g)) & 127;
        uint32_t sg = s7 | ((uint32_t)(__builtin_popcount(s7) & 1) << 7);
        int idx = p[2 + sb * 8 + g * 2 + (j % 8) / 4];
        uint32_t q = (uqo_iq3_grid(idx) >> (8 * (j % 4))) & 255;
        float scale = uqo_half(rd16(p)) * (0.5f + (float)(aux >> 28)) * 0.5f;
        return (scale * (float)q) * ((sg & (1u << (j % 8))) ? -1.0f : 1.0f);
    }
    }
    return NAN;
}

int uqo_dequantize(uint32_t kind, const uint8_t* in, int64_t n, float* out) {
    if (uqo_row_bytes(kind, n) < 0) return -1;
    for (int64_t i = 0; i < n; i++) {
        switch (kind) {
        case UQO_F32: { float v; memcpy(&v, in + 4 * i, 4); out[i] = v; break; }
        case UQO_Q8_0: {
            const uint8_t* p = in + (i / 32) * 34;
            out[i] = uqo_half(rd16(p)) * (float)(int8_t)p[2 + i % 32];
            break;
        }
        case UQO_Q4_K: {
            const uint8_t* p = in + (i / 256) * 144;
            int j = (int)(i % 256), sub = j / 32, sc, m;
            q4k_scale_min(sub, p + 4, &sc, &m);
            float d1 = uqo_half(rd16(p)) * (float)sc, m1 = uqo_half(rd16(p + 2)) * (float)m;
            out[i] = d1 * (float)q4k_value(j, p) - m1;
            break;
        }
        case UQO_Q3_K: {
            const uint8_t* p = in + (i / 256) * 110;
            int j = (int)(i % 256);
            float dl = uqo_half(rd16(p + 108)) * (float)(q3k_scale(j / 16, p + 96) - 32);
            out[i] = dl * (float)q3k_value(j, p);
            break;
        }
        default: out[i] = dequant_one(kind, in, i); break;
        }
    }
    return 0;
}

/* driver/kernels/gpu_dp4a.cu:23-31 (CPU form driver/src/gpu_prefill.rs:104-106):
 * per 32 values a = max|x|, inv = a>0 ? 127/a : 0, q = rint(x*inv) clamped to
 * +-127 (round half to even, __float2int_rn), scale = a/127. NaN quantizes to 0. */
void uqo_quant_act(const float* x, int64_t n, float* scale, int8_t* q) {
    for (int64_t b = 0; b < n / 32; b++) {
        float a = 0.0f;
        for (int j = 0; j < 32; j++) a = fmaxf(a, fabsf(x[b * 32 + j]));
        float inv = a > 0.0f ? 127.0f / a : 0.0f;
        for (int j = 0; j < 32; j++) {
            float v = x[b * 32 + j] * inv;
            float r = rintf(v);
            if (r != r) r = 0.0f;
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            q[b * 32 + j] = (int8_t)r;
        }
        scale[b] = a / 127.0f;
    }
}

static inline int32_t dot32(const int8_t* a, const int8_t* b) {
    int32_t s = 0;
    for (int j = 0; j < 32; j++) s += (int32_t)a[j] * (int32_t)b[j];
    return s;
}

/* Per-32-block int32 dots of a Q8_0 row with int8 activations
 * (gpu_dp4a.cu:43-47; gpu_prefill.rs:111-115). dots[row * (n/32) + block]. */
void uqo_q8_block_dots(const uint8_t* w, int64_t n, int64_t m, const int8_t* qx, int32_t* dots) {
    const int64_t nb = n / 32;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; r++)
        for (int64_t b = 0; b < nb; b++)
            dots[r * nb + b] = dot32((const int8_t*)(w + (r * nb + b) * 34 + 2), qx + b * 32);
}
/* Q4_K: per 32-value sub-block, sum of q(0..15) * qx. dots[row * (n/32) + sub]. */
void uqo_q4k_block_dots(const uint8_t* w, int64_t n, int64_t m, const int8_t* qx, int32_t* dots) {
    const int64_t nsb = n / 256;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; r++)
        for (int64_t s = 0; s < nsb; s++) {
            const uint8_t* p = w + (r * nsb + s) * 144;
            for (int a = 0; a < 8; a++) {
                int32_t acc = 0;
                for (int l = 0; l < 32; l++) acc += q4k_value(a * 32 + l, p) * qx[s * 256 + a * 32 + l];
                dots[r * (n / 32) + s * 8 + a] = acc;
            }
        }
}
/* Q3_K: per 16-value sub-block, sum of q3(-4..3) * qx. dots[row * (n/16) + sub]. */
void uqo_q3k_block_dots(const uint8_t* w, int64_t n, int64_t m, const int8_t* qx, int32_t* dots) {
    const int64_t nsb = n / 256;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; r++)
        for (int64_t s = 0; s < nsb; s++) {
            const uint8_t* p = w + (r * nsb + s) * 110;
            for (int a = 0; a < 16; a++) {
                int32_t acc = 0;
                for (int l = 0; l < 16; l++) acc += q3k_value(a * 16 + l, p) * qx[s * 256 + a * 16 + l];
                dots[r * (n / 16) + s * 16 + a] = acc;
            }
        }
}

/* One output of the decode matvec. Q8_0: y = sum_b dot_b * (dw_b * dx_b)
 * (gpu_dp4a.cu:47; gpu_prefill.rs:116) with the f32 product dw*dx as in the
 * reference; each term dot_b * (dw*dx) is exact in double (19 + 24 bits), the
 * terms are summed in double and rounded to f32 once.
 * Q4_K (ggml): term per 32-block a = dx_a * ((d*sc) * isum - (dmin*m) * xsum).
 * Q3_K (ggml): term per 32-block a = dx_a * ((d*(sc0-32)) * isum0 + (d*(sc1-32)) * isum1). */
static float matvec_row(uint32_t kind, const uint8_t* row, int64_t n, const float* xs, const int8_t* qx) {
    double acc = 0.0;
    if (kind == UQO_Q8_0) {
        for (int64_t b = 0; b < n / 32; b++) {
            const uint8_t* p = row + b * 34;
            int32_t c = dot32((const int8_t*)(p + 2), qx + b * 32);
            float s = uqo_half(rd16(p)) * xs[b];
            acc += (double)c * (double)s;
        }
    } else if (kind == UQO_Q4_K) {
        for (int64_t sb = 0; sb < n / 256; sb++) {
            const uint8_t* p = row + sb * 144;
            const float d = uqo_half(rd16(p)), dmin = uqo_half(rd16(p + 2));
            for (int a = 0; a < 8; a++) {
                int sc, m;
                q4k_scale_min(a, p + 4, &sc, &m);
                const int8_t* xq = qx + sb * 256 + a * 32;
                int32_t isum = 0, xsum = 0;
                for (int l = 0; l < 32; l++) { isum += q4k_value(a * 32 + l, p) * xq[l]; xsum += xq[l]; }
                const float d1 = d * (float)sc, m1 = dmin * (float)m;
                const double inner = (double)d1 * (double)isum - (double)m1 * (double)xsum;
                acc += (double)xs[sb * 8 + a] * inner;
            }
        }
    } else if (kind == UQO_Q3_K) {
        for (int64_t sb = 0; sb < n / 256; sb++) {
            const uint8_t* p = row + sb * 110;
            const float d = uqo_half(rd16(p + 108));
            for (int a = 0; a < 8; a++) {
                const int8_t* xq = qx + sb * 256 + a * 32;
                int32_t i0 = 0, i1 = 0;
                for (int l = 0; l < 16; l++) {
                    i0 += q3k_value(a * 32 + l, p) * xq[l];
                    i1 += q3k_value(a * 32 + 16 + l, p) * xq[16 + l];
                }
                const float dl0 = d * (float)(q3k_scale(2 * a, p + 96) - 32);
                const float dl1 = d * (float)(q3k_scale(2 * a + 1, p + 96) - 32);
                const double inner = (double)dl0 * (double)i0 + (double)dl1 * (double)i1;
                acc += (double)xs[sb * 8 + a] * inner;
            }
        }
    }
    return (float)acc;
}

/* Decode matvec y = W x with int8 activations (linear_dp4a, gpu_dp4a.cu:40-52;
 * host graph_linear, gpu_graph.rs:74-80). n = K (columns), m = N (rows). */
void uqo_matvec(uint32_t kind, const uint8_t* w, int64_t n, int64_t m,
                const float* xscale, const int8_t* qx, float* y) {
    const int64_t rb = uqo_row_bytes(kind, n);
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; r++) y[r] = matvec_row(kind, w + r * rb, n, xscale, qx);
}

/* Gpu::matvec semantics (llm.rs:246-273) with the graph's int8 activations:
 * quantize x per 32 (uqo_quant_act) then uqo_matvec. */
void uqo_matvec_x(uint32_t kind, const uint8_t* w, int64_t n, int64_t m, const float* x, float* y) {
    float* xs = (float*)malloc(sizeof(float) * (size_t)(n / 32));
    int8_t* qx = (int8_t*)malloc((size_t)n);
    uqo_quant_act(x, n, xs, qx);
    uqo_matvec(kind, w, n, m, xs, qx, y);
    free(xs); free(qx);
}

/* The literal CPU check of driver/src/gpu_prefill.rs:104-116: quantize, then
 * expect += dot as f32 * (d * scale) in f32, sequentially over blocks. */
void uqo_q8_matvec_f32seq(const uint8_t* w, int64_t n, int64_t m, const float* x, float* y) {
    const int64_t nb = n / 32;
    float* xs = (float*)malloc(sizeof(float) * (size_t)nb);
    int8_t* qx = (int8_t*)malloc((size_t)n);
    uqo_quant_act(x, n, xs, qx);
    for (int64_t r = 0; r < m; r++) {
        float expect = 0.0f;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t* p = w + (r * nb + b) * 34;
            int32_t c = dot32((const int8_t*)(p + 2), qx + b * 32);
            float s = uqo_half(rd16(p)) * xs[b];
            float t = (float)c * s;
            expect = expect + t;
        }
        y[r] = expect;
    }
    free(xs); free(qx);
}

/* driver/src/llm.rs:302-309: fp32 dequant dot, expect += q8(row,col) * x[col]. */
void uqo_q8_dequant_dot(const uint8_t* w, int64_t n, int64_t m, const float* x, float* y) {
    const int64_t nb = n / 32;
    for (int64_t r = 0; r < m; r++) {
        float expect = 0.0f;
        for (int64_t c = 0; c < n; c++) {
            const uint8_t* p = w + (r * nb + c / 32) * 34;
            float wv = uqo_half(rd16(p)) * (float)(int8_t)p[2 + c % 32];
            float t = wv * x[c];
            expect = expect + t;
        }
        y[r] = expect;
    }
}

/* Q8_0 prefill GEMM (driver/kernels/gpu_prefill.cu:10-36; oracle
 * gpu_prefill.rs:95-121): per 32-block int32 dot, accumulator reset per block,
 * f = fmaf((float)c, dw * dx, f) sequentially over blocks. y[token * m + row]. */
void uqo_prefill_gemm(const uint8_t* w, int64_t n, int64_t m, int64_t batch,
                      const float* xscale, const int8_t* qx, float* y) {
    const int64_t nb = n / 32;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; r++) {
        const uint8_t* row = w + r * nb * 34;
        for (int64_t t = 0; t < batch; t++) {
            float f = 0.0f;
            for (int64_t b = 0; b < nb; b++) {
                const uint8_t* p = row + b * 34;
                int32_t c = dot32((const int8_t*)(p + 2), qx + t * n + b * 32);
                float s = uqo_half(rd16(p)) * xscale[t * nb + b];
                f = fmaf((float)c, s, f);
            }
            y[t * m + r] = f;
        }
    }
}

/* RMSNorm: driver/kernels/gpu_fused.cu:28-35 (y = x * scale * w, eps 1e-6)
 * with the sum of squares formed as in driver/src/frontier_forward.rs:38-42:
 * f32 squares summed in double, mean rounded to f32. */
void uqo_rmsnorm(const float* x, const float* gamma, int64_t n, float eps, float* y) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; i++) { float sq = x[i] * x[i]; sum += (double)sq; }
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; i++) { float t = x[i] * scale; y[i] = t * gamma[i]; }
}

/* driver/src/gpu_graph.rs:131-133: per position, cos in [0, hd/2) and sin in
 * [hd/2, hd): angle = pos * powf(theta, -(2i)/hd). */
void uqo_rope_table(int seq, int head_dim, float theta, float* table) {
    const int half = head_dim / 2;
    for (int pos = 0; pos < seq; pos++)
        for (int i = 0; i < half; i++) {
            float e = -((float)(2 * i)) / (float)head_dim;
            float angle = (float)pos * powf(theta, e);
            float s, c;
            sincosf(angle, &s, &c);
            table[pos * head_dim + i] = c;
            table[pos * head_dim + half + i] = s;
        }
}

/* driver/kernels/gpu_ops.cu:9-20: bias add then NeoX rotate-half on pairs
 * (j, j+hd/2): u = v[a]+b[a], w = v[b]+b[b]; v[a] = u*c - w*s; v[b] = u*s + w*c. */
void uqo_rope_bias(float* v, const float* bias, int heads, int head_dim, const float* trig_row) {
    const int half = head_dim / 2;
    for (int h = 0; h < heads; h++)
        for (int j = 0; j < half; j++) {
            const int a = h * head_dim + j, b = a + half;
            const float cs = trig_row[j], sn = trig_row[half + j];
            float u = bias ? v[a] + bias[a] : v[a];
            float w = bias ? v[b] + bias[b] : v[b];
            float p0 = u * cs, p1 = w * sn, p2 = u * sn, p3 = w * cs;
            v[a] = p0 - p1;
            v[b] = p2 + p3;
        }
}

/* driver/kernels/gpu_dp4a.cu:63 (and gpu_ops.cu:41): (g / (1 + exp(-g))) * u. */
float uqo_silu_mul(float g, float u) {
    float e = uqo_expf(-g);
    float den = 1.0f + e;
    float s = g / den;
    return s * u;
}

/* Decode attention, driver/kernels/gpu_attention.cu:2-26 (CPU form
 * llm.rs:355-368) over an fp16 KV cache laid out [t][kv_heads*hd]:
 * s_t = (q.k_t) * (1/sqrt(hd)) with q.k summed in double; softmax with max
 * subtraction, e_t = exp(s_t - max), total summed in double, p_t = e_t/total;
 * out = sum_t p_t v_t summed in double. Query head h reads KV head h/(heads/kv). */
void uqo_attention(const float* q, const uint16_t* keys, const uint16_t* values, int pos,
                   int heads, int kv_heads, int head_dim, float* out) {
    const int kvd = kv_heads * head_dim, group = heads / kv_heads, T = pos + 1;
    const float qscale = (float)(1.0 / sqrt((double)head_dim));
    float* sc = (float*)malloc(sizeof(float) * (size_t)T);
    for (int h = 0; h < heads; h++) {
        const int kh = h / group;
        const float* qh = q + h * head_dim;
        float mx = -FLT_MAX;
        for (int t = 0; t < T; t++) {
            const uint16_t* k = keys + (size_t)t * kvd + kh * head_dim;
            double acc = 0.0;
            for (int d = 0; d < head_dim; d++) acc += (double)qh[d] * (double)uqo_half(k[d]);
            sc[t] = (float)acc * qscale;
            mx = fmaxf(mx, sc[t]);
        }
        double tot = 0.0;
        for (int t = 0; t < T; t++) { sc[t] = uqo_expf(sc[t] - mx); tot += (double)sc[t]; }
        const float total = (float)tot;
        for (int t = 0; t < T; t++) sc[t] = sc[t] / total;
        for (int d = 0; d < head_dim; d++) {
            double acc = 0.0;
            for (int t = 0; t < T; t++)
                acc += (double)sc[t] * (double)uqo_half(values[(size_t)t * kvd + kh * head_dim + d]);
            out[h * head_dim + d] = (float)acc;
        }
    }
    free(sc);
}

/* driver/kernels/gpu_greedy.cu:1-27 (CPU check gpu_graph.rs:14-23): argmax,
 * the lowest id wins ties, any non-finite logit marks the result bad. */
int uqo_greedy(const float* logits, int64_t n, int* bad) {
    float best = -INFINITY;
    int64_t id = 0x7fffffff;
    int b = 0;
    for (int64_t i = 0; i < n; i++) {
        float v = logits[i];
        if ((bits_from_f(v) & 0x7f800000u) == 0x7f800000u) b = 1;
        if (v > best || (v == best && i < id)) { best = v; id = i; }
    }
    if (bad) *bad = b;
    return (int)id;
}

/* ----------------------------------------------------------------------- */
/* Qwen2 dense decoder.                                                     */

struct uqo_state {
    uqo_qwen2 m;
    uint16_t* keys;   /* [layers][max_seq][kv_dim] */
    uint16_t* values;
    float* trig;      /* [max_seq][head_dim] */
};

uqo_state* uqo_state_new(const uqo_qwen2* m) {
    uqo_state* s = (uqo_state*)calloc(1, sizeof(uqo_state));
    s->m = *m;
    const size_t kv = (size_t)m->layers * m->max_seq * m->kv_heads * m->head_dim;
    s->keys = (uint16_t*)calloc(kv, 2);
    s->values = (uint16_t*)calloc(kv, 2);
    s->trig = (float*)malloc(sizeof(float) * (size_t)m->max_seq * m->head_dim);
    uqo_rope_table(m->max_seq, m->head_dim, m->theta, s->trig);
    return s;
}
void uqo_state_free(uqo_state* s) {
    if (!s) return;
    free(s->keys); free(s->values); free(s->trig); free(s);
}
const uint16_t* uqo_state_keys(const uqo_state* s, int layer) {
    return s->keys + (size_t)layer * s->m.max_seq * s->m.kv_heads * s->m.head_dim;
}
const uint16_t* uqo_state_values(const uqo_state* s, int layer) {
    return s->values + (size_t)layer * s->m.max_seq * s->m.kv_heads * s->m.head_dim;
}

/* embedding_q8, driver/kernels/gpu_embedding.cu:3-9: x = half(d) * q. */
static void embed(const uqo_qwen2* m, uint32_t token, float* x) {
    const int64_t nb = m->dim / 32;
    for (int i = 0; i < m->dim; i++) {
        const uint8_t* p = m->tok_embd + ((int64_t)token * nb + i / 32) * 34;
        x[i] = uqo_half(rd16(p)) * (float)(int8_t)p[2 + i % 32];
    }
}

static int all_finite(const float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) if (!isfinite(x[i])) return 0;
    return 1;
}

/* Output head: fused_resnorm(X += TMP) with output_norm, quant, lm_head matvec,
 * greedy (gpu_graph.rs:158-162). x already holds the summed residual. */
static int head(const uqo_qwen2* m, const float* x, uint32_t* next, float* logits_out) {
    float* xn = (float*)malloc(sizeof(float) * m->dim);
    float* xs = (float*)malloc(sizeof(float) * (m->dim / 32));
    int8_t* xq = (int8_t*)malloc(m->dim);
    float* logits = logits_out ? logits_out : (float*)malloc(sizeof(float) * (size_t)m->vocab);
    uqo_rmsnorm(x, m->output_norm, m->dim, m->eps, xn);
    uqo_quant_act(xn, m->dim, xs, xq);
    uqo_matvec(UQO_Q8_0, m->output, m->dim, m->vocab, xs, xq, logits);
    int bad = 0;
    int id = uqo_greedy(logits, m->vocab, &bad);
    if (next) *next = (uint32_t)id;
    if (!logits_out) free(logits);
    free(xn); free(xs); free(xq);
    return bad ? -1 : 0;
}

/* One decode step at position pos (gpu_graph.rs:137-162 job order; CPU form
 * llm.rs:339-388). */
int uqo_decode(uqo_state* s, uint32_t token, int pos, uint32_t* next, float* logits) {
    const uqo_qwen2* m = &s->m;
    if (pos < 0 || pos >= m->max_seq || (int64_t)token >= m->vocab) return -2;
    const int D = m->dim, H = m->hidden, hd = m->head_dim, kvd = m->kv_heads * hd;
    float *x = malloc(sizeof(float) * D), *tmp = malloc(sizeof(float) * D), *xn = malloc(sizeof(float) * D);
    float *q = malloc(sizeof(float) * D), *k = malloc(sizeof(float) * kvd), *v = malloc(sizeof(float) * kvd);
    float *att = malloc(sizeof(float) * D), *g = malloc(sizeof(float) * H), *u = malloc(sizeof(float) * H);
    float *xs = malloc(sizeof(float) * (H / 32));
    int8_t* xq = malloc(H);
    int rc = 0;
    embed(m, token, x);
    const float* trig = s->trig + (size_t)pos * hd;
    for (int l = 0; l < m->layers; l++) {
        const uqo_layer* L = &m->layer[l];
        if (l > 0) for (int i = 0; i < D; i++) x[i] = x[i] + tmp[i];
        uqo_rmsnorm(x, L->attn_norm, D, m->eps, xn);
        uqo_quant_act(xn, D, xs, xq);
        uqo_matvec(UQO_Q8_0, L->wq, D, D, xs, xq, q);
        uqo_matvec(UQO_Q8_0, L->wk, D, kvd, xs, xq, k);
        uqo_matvec(UQO_Q8_0, L->wv, D, kvd, xs, xq, v);
        uqo_rope_bias(q, L->bq, m->heads, hd, trig);
        uqo_rope_bias(k, L->bk, m->kv_heads, hd, trig);
        uint16_t* kc = (uint16_t*)uqo_state_keys(s, l) + (size_t)pos * kvd;
        uint16_t* vc = (uint16_t*)uqo_state_values(s, l) + (size_t)pos * kvd;
        for (int i = 0; i < kvd; i++) {
            kc[i] = uqo_f16_rne(k[i]);
            float vb = L->bv ? v[i] + L->bv[i] : v[i];
            vc[i] = uqo_f16_rne(vb);
        }
        uqo_attention(q, uqo_state_keys(s, l), uqo_state_values(s, l), pos, m->heads, m->kv_heads, hd, att);
        uqo_quant_act(att, D, xs, xq);
        uqo_matvec(UQO_Q8_0, L->wo, D, D, xs, xq, tmp);
        for (int i = 0; i < D; i++) x[i] = x[i] + tmp[i];
        uqo_rmsnorm(x, L->ffn_norm, D, m->eps, xn);
        uqo_quant_act(xn, D, xs, xq);
        uqo_matvec(UQO_Q8_0, L->wg, D, H, xs, xq, g);
        uqo_matvec(UQO_Q8_0, L->wu, D, H, xs, xq, u);
        for (int i = 0; i < H; i++) g[i] = uqo_silu_mul(g[i], u[i]);
        uqo_quant_act(g, H, xs, xq);
        uqo_matvec(UQO_Q8_0, L->wd, H, D, xs, xq, tmp);
        if (!all_finite(tmp, D)) { rc = -3; goto done; }
    }
    for (int i = 0; i < D; i++) x[i] = x[i] + tmp[i];
    rc = head(m, x, next, logits);
done:
    free(x); free(tmp); free(xn); free(q); free(k); free(v); free(att); free(g); free(u); free(xs); free(xq);
    return rc;
}

/* Prompt prefill over positions 0..count-1 (gpu_prefill.rs:122-150 job order):
 * all linears run as the Q8_0 prefill GEMM; the last token's residual feeds the
 * decode output head (gpu_prefill.rs:138-148). */
int uqo_prefill(uqo_state* s, const uint32_t* tokens, int count, uint32_t* next, float* logits) {
    const uqo_qwen2* m = &s->m;
    if (count <= 0 || count > m->max_seq) return -2;
    for (int t = 0; t < count; t++) if ((int64_t)tokens[t] >= m->vocab) return -2;
    const int64_t n = count;
    const int D = m->dim, H = m->hidden, hd = m->head_dim, kvd = m->kv_heads * hd;
    float *X = malloc(sizeof(float) * n * D), *TMP = malloc(sizeof(float) * n * D);
    float *XN = malloc(sizeof(float) * n * H), *Q = malloc(sizeof(float) * n * D);
    float *K = malloc(sizeof(float) * n * kvd), *V = malloc(sizeof(float) * n * kvd);
    float *G = malloc(sizeof(float) * n * H), *U = malloc(sizeof(float) * n * H);
    float *XS = malloc(sizeof(float) * n * (H / 32));
    int8_t* XQ = malloc((size_t)n * H);
    int rc = 0;
    for (int64_t t = 0; t < n; t++) embed(m, tokens[t], X + t * D);
    for (int l = 0; l < m->layers; l++) {
        const uqo_layer* L = &m->layer[l];
        uint16_t* kc = (uint16_t*)uqo_state_keys(s, l);
        uint16_t* vc = (uint16_t*)uqo_state_values(s, l);
        #pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < n; t++) {
            if (l > 0) for (int i = 0; i < D; i++) X[t * D + i] = X[t * D + i] + TMP[t * D + i];
            uqo_rmsnorm(X + t * D, L->attn_norm, D, m->eps, XN + t * D);
            uqo_quant_act(XN + t * D, D, XS + t * (D / 32), XQ + t * D);
        }
        uqo_prefill_gemm(L->wq, D, D, n, XS, XQ, Q);
        uqo_prefill_gemm(L->wk, D, kvd, n, XS, XQ, K);
        uqo_prefill_gemm(L->wv, D, kvd, n, XS, XQ, V);
        #pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < n; t++) {
            const float* trig = s->trig + (size_t)t * hd;
            uqo_rope_bias(Q + t * D, L->bq, m->heads, hd, trig);
            uqo_rope_bias(K + t * kvd, L->bk, m->kv_heads, hd, trig);
            for (int i = 0; i < kvd; i++) {
                kc[t * kvd + i] = uqo_f16_rne(K[t * kvd + i]);
                float vb = L->bv ? V[t * kvd + i] + L->bv[i] : V[t * kvd + i];
                vc[t * kvd + i] = uqo_f16_rne(vb);
            }
        }
        #pragma omp parallel for schedule(dynamic, 4)
        for (int64_t t = 0; t < n; t++) {
            uqo_attention(Q + t * D, kc, vc, (int)t, m->heads, m->kv_heads, hd, XN + t * D);
            uqo_quant_act(XN + t * D, D, XS + t * (D / 32), XQ + t * D);
        }
        uqo_prefill_gemm(L->wo, D, D, n, XS, XQ, TMP);
        #pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < n; t++) {
            for (int i = 0; i < D; i++) X[t * D + i] = X[t * D + i] + TMP[t * D + i];
            uqo_rmsnorm(X + t * D, L->ffn_norm, D, m->eps, XN + t * D);
            uqo_quant_act(XN + t * D, D, XS + t * (D / 32), XQ + t * D);
        }
        uqo_prefill_gemm(L->wg, D, H, n, XS, XQ, G);
        uqo_prefill_gemm(L->wu, D, H, n, XS, XQ, U);
        #pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < n; t++) {
            for (int i = 0; i < H; i++) G[t * H + i] = uqo_silu_mul(G[t * H + i], U[t * H + i]);
            uqo_quant_act(G + t * H, H, XS + t * (H / 32), XQ + t * H);
        }
        uqo_prefill_gemm(L->wd, H, D, n, XS, XQ, TMP);
        if (!all_finite(TMP, n * D)) { rc = -3; goto done; }
    }
    {
        float* x = X + (n - 1) * D;
        const float* tl = TMP + (n - 1) * D;
        for (int i = 0; i < D; i++) x[i] = x[i] + tl[i];
        rc = head(m, x, next, logits);
    }
done:
    free(X); free(TMP); free(XN); free(Q); free(K); free(V); free(G); free(U); free(XS); free(XQ);
    return rc;
}

/* ----------------------------------------------------------------------- */
/* MoE expert FFN, driver/src/frontier_forward.rs:164-199.                   */

/* frontier_forward.rs:47-51 softmax (max fold, exp, f32 running sum, divide),
 * then :167 stable order (score descending, id ascending), top-k, :168 the
 * f32 sum of the selected scores, weights score/sum (:191). */
int uqo_moe_route(const float* logits, int experts, int top_k, int32_t* ids, float* weights) {
    if (experts <= 0 || top_k <= 0 || top_k > experts) return -2;
    if (!all_finite(logits, experts)) return -3;
    float* p = (float*)malloc(sizeof(float) * experts);
    float mx = -INFINITY;
    for (int e = 0; e < experts; e++) mx = fmaxf(mx, logits[e]);
    float sum = 0.0f;
    for (int e = 0; e < experts; e++) { p[e] = uqo_expf(logits[e] - mx); sum = sum + p[e]; }
    if (!(sum > 0.0f) || !isfinite(sum)) { free(p); return -3; }
    for (int e = 0; e < experts; e++) p[e] = p[e] / sum;
    /* selection by repeated scan = the prefix of a stable (desc score, asc id) sort */
    unsigned char* used = (unsigned char*)calloc(experts, 1);
    for (int k = 0; k < top_k; k++) {
        int best = -1;
        for (int e = 0; e < experts; e++) {
            if (used[e]) continue;
            if (best < 0 || p[e] > p[best]) best = e;
        }
        used[best] = 1;
        ids[k] = best;
    }
    float tot = 0.0f;
    for (int k = 0; k < top_k; k++) tot = tot + p[ids[k]];
    int rc = 0;
    if (!(tot > 0.0f)) rc = -3;
    for (int k = 0; k < top_k; k++) weights[k] = p[ids[k]] / tot;
    free(p); free(used);
    return rc;
}

/* frontier_cpu_expf.rs:12-19: activation(x, silu): v = 1/(1+exp(-x)); silu = x*v. */
static float act_sigmoid(float x) { float e = uqo_expf(-x); float d = 1.0f + e; return 1.0f / d; }

/* frontier_forward.rs:164-199 with int8 activations per 32 for every expert
 * matvec: per selected expert down(silu(gate x) * (up x)); shared expert the
 * same; out = sum over rank order of weight*value (frontier_cpu_axpy.rs:13-21,
 * separate multiply then add), then += sigmoid(shexp_gate . x) * shared
 * (weight 1 when sh_scale is NULL: no ffn_gate_inp_shexp tensor). */
int uqo_moe_ffn(const uqo_moe* mo, const float* x, const float* router_logits, float* out,
                int32_t* ids_out, float* weights_out) {
    const int D = mo->dim, F = mo->ff, K = mo->top_k;
    int32_t ids[64];
    float wts[64];
    if (K > 64) return -2;
    int rc = uqo_moe_route(router_logits, mo->experts, K, ids, wts);
    if (rc) return rc;
    if (!all_finite(x, D)) return -3;
    float *xs = malloc(sizeof(float) * (D / 32)), *fs = malloc(sizeof(float) * (F / 32));
    int8_t *xq = malloc(D), *fq = malloc(F);
    float *g = malloc(sizeof(float) * F), *u = malloc(sizeof(float) * F), *val = malloc(sizeof(float) * D);
    uqo_quant_act(x, D, xs, xq);
    for (int i = 0; i < D; i++) out[i] = 0.0f;
    for (int k = 0; k <= K; k++) {
        const int shared = (k == K);
        const uint32_t kind = shared ? mo->shared_kind : mo->expert_kind;
        const uint8_t* wg = shared ? mo->sh_gate : mo->gate[ids[k]];
        const uint8_t* wu = shared ? mo->sh_up : mo->up[ids[k]];
        const uint8_t* wd = shared ? mo->sh_down : mo->down[ids[k]];
        uqo_matvec(kind, wg, D, F, xs, xq, g);
        uqo_matvec(kind, wu, D, F, xs, xq, u);
        for (int i = 0; i < F; i++) { float sg = g[i] * act_sigmoid(g[i]); g[i] = sg * u[i]; }
        uqo_quant_act(g, F, fs, fq);
        uqo_matvec(kind, wd, F, D, fs, fq, val);
        if (!all_finite(val, D)) { rc = -3; break; }
        float weight;
        if (shared && mo->sh_scale) {
            double acc = 0.0;
            for (int i = 0; i < D; i++) acc += (double)mo->sh_scale[i] * (double)x[i];
            weight = act_sigmoid((float)acc);
        } else if (shared) {
            weight = 1.0f;              /* a model without ffn_gate_inp_shexp: the shared expert unscaled */
        } else {
            weight = wts[k];
        }
        for (int i = 0; i < D; i++) { float t = weight * val[i]; out[i] = out[i] + t; }
    }
    if (ids_out) for (int k = 0; k < K; k++) ids_out[k] = ids[k];
    if (weights_out) for (int k = 0; k < K; k++) weights_out[k] = wts[k];
    free(xs); free(fs); free(xq); free(fq); free(g); free(u); free(val);
    if (!rc && !all_finite(out, D)) rc = -3;
    return rc;
}

/* ---------------------------------------------------------------- fp32-activation reader
 * frontier_matvec (frontier_quant.cu:58-66; host Weights::linear,
 * frontier_backend.rs:243): y[r] = sum_i value(r, i) * x[i] with fp32 x. Each
 * value is a dequantize() f32 whose products with x are exact in double; the
 * sum runs in double in index order and is rounded to f32 once. */
void uqo_linear(uint32_t kind, const uint8_t* w, int64_t n, int64_t m, const float* x, float* y) {
    const int64_t rb = uqo_row_bytes(kind, n);
    #pragma omp parallel
    {
        float* v = (float*)malloc(sizeof(float) * (size_t)n);
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < m; r++) {
            uqo_dequantize(kind, w + r * rb, n, v);
            double acc = 0.0;
            for (int64_t i = 0; i < n; i++) acc += (double)v[i] * (double)x[i];
            y[r] = (float)acc;
        }
        free(v);
    }
}

/* The reference's own CPU check of frontier_matvec (frontier_gpu.rs:104,
 * :176-178): reference += dequant[j] * x[j] in f32, sequentially, multiply
 * then add. Its tolerance is 2e-4 + 2e-5 |reference| (:111). */
void uqo_linear_f32seq(uint32_t kind, const uint8_t* w, int64_t n, int64_t m, const float* x, float* y) {
    const int64_t rb = uqo_row_bytes(kind, n);
    float* v = (float*)malloc(sizeof(float) * (size_t)n);
    for (int64_t r = 0; r < m; r++) {
        uqo_dequantize(kind, w + r * rb, n, v);
        float acc = 0.0f;
        for (int64_t i = 0; i < n; i++) {
            float t = v[i] * x[i];
            acc = acc + t;
        }
        y[r] = acc;
    }
    free(v);
}

/* The reference's synthetic quant bytes, frontier_gpu.rs:37-50: xorshift32
 * bytes from state 0x13243546 (<<13, >>17, <<5, low byte), F32/BF16 values
 * ((i % 127) - 63) / 64, and each block's fp16 scale field set to
 * 0x2000, 0x2800, 0x3000, 0xb000 in turn. Returns bytes written or <0. */
int64_t uqo_frontier_fixture(uint32_t kind, int64_t n, uint8_t* out) {
    const int64_t rb = uqo_row_bytes(kind, n);
    if (rb < 0) return -1;
    uint32_t st = 0x13243546u;
    for (int64_t i = 0; i < rb; i++) {
        st ^= st << 13;
        st ^= st >> 17;
        st ^= st << 5;
        out[i] = (uint8_t)st;
    }
    if (kind == UQO_F32 || kind == UQO_BF16) {
        for (int64_t i = 0; i < n; i++) {
            uint32_t bits = bits_from_f(((float)(i % 127) - 63.0f) / 64.0f);
            if (kind == UQO_F32) memcpy(out + 4 * i, &bits, 4);
            else { uint16_t h = (uint16_t)(bits >> 16); memcpy(out + 2 * i, &h, 2); }
        }
    } else {
        int64_t block, size, off;
        switch (kind) {
        case UQO_Q8_0: block = 32; size = 34; off = 0; break;
        case UQO_Q6_K: block = 256; size = 210; off = 208; break;
        case UQO_IQ3_XXS: block = 256; size = 98; off = 0; break;
        case UQO_IQ4_NL: block = 32; size = 18; off = 0; break;
        case UQO_IQ4_XS: block = 256; size = 136; off = 0; break;
        default: return -2;
        }
        static const uint16_t halves[4] = {0x2000, 0x2800, 0x3000, 0xb000};
        for (int64_t b = 0; b < n / block; b++) {
            uint16_t h = halves[b % 4];
            memcpy(out + b * size + off, &h, 2);
        }
    }
    return rb;
}


/* ----------------------------------------------------------------------- */
/* Reference-order decode: the f32 operation orders of the reference's      */
/* decode graph (gpu_graph.rs:137-162), kernel by kernel. A second oracle   */
/* form beside the exact-double contract above, for tolerance-graded        */
/* comparison against the reference's own arithmetic:                       */
/*   embedding_q8        gpu_embedding.cu:3-9                               */
/*   fused_resnorm       gpu_fused.cu:28-35 (128-thread strided squares,    */
/*                       shared-memory tree 64..1, (v*scale)*w)             */
/*   quant_act           gpu_dp4a.cu:23-31 (= uqo_quant_act)                */
/*   qkv_dp4a/gateup     gpu_dp4a.cu:32-39,53-64 (dotrow: 32 lanes, 8-byte   */
/*                       segments, fmaf per block, xor butterfly 16..1)     */
/*   linear_dp4a         gpu_dp4a.cu:40-52 (128 threads, 16-byte halves,    */
/*                       fmaf per half-block, warp butterflies, then        */
/*                       ((p0+p1)+p2)+p3)                                    */
/*   rope_bias           gpu_ops.cu:9-20 (shared host trig table)           */
/*   fused_attention     gpu_attention.cu:2-26 (f32 KV; lane-strided q.k    */
/*                       with butterfly, strided exp sums + tree, p/total,  */
/*                       sequential P.V)                                    */
/*   greedy              gpu_greedy.cu:1-27                                 */
/* Every multiply and add is a separate f32 rounding except the explicit    */
/* fmaf of the dp4a kernels (the reference builds with --fmad=false).       */
/* exp is uqo_expf (libm's algorithm) where the GPU kernels call CUDA's     */
/* expf, whose steps are not reproduced; that and the host trig table are   */
/* the only departures. kv_fp16 != 0 rounds cached K and V to fp16, the     */
/* library's cache format, to separate order effects from cache             */
/* precision.                                                               */

struct uqo_refo {
    uqo_qwen2 m;
    int kv_fp16;
    float* keys;   /* [layers][max_seq][kv_dim] */
    float* values;
    float* trig;
};

uqo_refo* uqo_refo_new(const uqo_qwen2* m, int kv_fp16) {
    uqo_refo* s = (uqo_refo*)calloc(1, sizeof(uqo_refo));
    s->m = *m;
    s->kv_fp16 = kv_fp16;
    const size_t kv = (size_t)m->layers * m->max_seq * m->kv_heads * m->head_dim;
    s->keys = (float*)calloc(kv, sizeof(float));
    s->values = (float*)calloc(kv, sizeof(float));
    s->trig = (float*)malloc(sizeof(float) * (size_t)m->max_seq * m->head_dim);
    uqo_rope_table(m->max_seq, m->head_dim, m->theta, s->trig);
    return s;
}
void uqo_refo_free(uqo_refo* s) {
    if (!s) return;
    free(s->keys); free(s->values); free(s->trig); free(s);
}

/* xor butterfly of a 32-lane warp (x += shfl_xor(x, 16); ... 1): lane 0's total. */
static float refo_butterfly32(float* v) {
    for (int off = 16; off; off >>= 1) {
        float t[32];
        for (int i = 0; i < 32; i++) t[i] = v[i] + v[i ^ off];
        memcpy(v, t, sizeof(t));
    }
    return v[0];
}

/* fused_resnorm, gpu_fused.cu:28-35, for n values (the kernel's n is 1536). */
void uqo_refo_resnorm(float* x, const float* residual, const float* w, float* y, int n, float eps, int add) {
    float sums[128];
    for (int t = 0; t < 128; t++) {
        float sum = 0.0f;
        for (int i = t; i < n; i += 128) {
            float v = add ? x[i] + residual[i] : x[i];
            float sq = v * v;
            sum = sum + sq;
        }
        sums[t] = sum;
    }
    for (int stride = 64; stride; stride >>= 1)
        for (int t = 0; t < stride; t++) sums[t] = sums[t] + sums[t + stride];
    const float mean = sums[0] / (float)n;
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < n; i++) {
        float v = add ? x[i] + residual[i] : x[i];
        if (add) x[i] = v;
        float t = v * scale;
        y[i] = t * w[i];
    }
}

static int32_t dp4a8(const int8_t* a, const int8_t* b, int n) {
    int32_t s = 0;
    for (int j = 0; j < n; j++) s += (int32_t)a[j] * (int32_t)b[j];
    return s;
}

/* dotrow, gpu_dp4a.cu:32-39: one 32-lane warp over a Q8_0 row of `blocks`
 * blocks; lane l takes bytes 8*(l&3).. of blocks l>>2, l>>2 + 8, ... */
float uqo_refo_dotrow(const uint8_t* w, const float* xs, const int8_t* xq, int64_t blocks) {
    float lanes[32];
    for (int lane = 0; lane < 32; lane++) {
        const int seg = lane & 3;
        float sum = 0.0f;
        for (int64_t b = lane >> 2; b < blocks; b += 8) {
            const uint8_t* wp = w + b * 34;
            const int32_t acc = dp4a8((const int8_t*)(wp + 2 + seg * 8), xq + b * 32 + seg * 8, 8);
            const float d = uqo_half(rd16(wp)) * xs[b];
            sum = fmaf((float)acc, d, sum);
        }
        lanes[lane] = sum;
    }
    return refo_butterfly32(lanes);
}

/* linear_dp4a, gpu_dp4a.cu:40-52: 128 threads per row; thread t takes the
 * 16-byte half (t&1) of blocks t>>1, t>>1 + 64, ...; warp butterflies, then
 * ((p0 + p1) + p2) + p3. */
float uqo_refo_linear_row(const uint8_t* w, const float* xs, const int8_t* xq, int64_t blocks) {
    float p[4];
    for (int warp = 0; warp < 4; warp++) {
        float lanes[32];
        for (int lane = 0; lane < 32; lane++) {
            const int tid = warp * 32 + lane, seg = tid & 1;
            float sum = 0.0f;
            for (int64_t b = tid >> 1; b < blocks; b += 64) {
                const uint8_t* wp = w + b * 34;
                const int32_t acc = dp4a8((const int8_t*)(wp + 2 + seg * 16), xq + b * 32 + seg * 16, 16);
                const float d = uqo_half(rd16(wp)) * xs[b];
                sum = fmaf((float)acc, d, sum);
            }
            lanes[lane] = sum;
        }
        p[warp] = refo_butterfly32(lanes);
    }
    const float a = p[0] + p[1];
    const float b = a + p[2];
    return b + p[3];
}

static void refo_linear(const uint8_t* w, int64_t n, int64_t m, const float* xs, const int8_t* xq, float* y) {
    const int64_t blocks = n / 32, rb = blocks * 34;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; r++) y[r] = uqo_refo_linear_row(w + r * rb, xs, xq, blocks);
}
static void refo_dotrows(const uint8_t* w, int64_t n, int64_t m, const float* xs, const int8_t* xq, float* y) {
    const int64_t blocks = n / 32, rb = blocks * 34;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; r++) y[r] = uqo_refo_dotrow(w + r * rb, xs, xq, blocks);
}

/* fused_attention, gpu_attention.cu:2-26, for one query head over f32 keys
 * and values [t][kvd] at KV head kh; head_dim hd (the kernel's is 128). */
void uqo_refo_attention_head(const float* q, const float* keys, const float* values, int pos, int kvd, int kh,
                             int hd, float* out) {
    const int T = pos + 1;
    float* scores = (float*)malloc(sizeof(float) * (size_t)T);
    const float qscale = (float)(1.0 / sqrt((double)hd));
    for (int t = 0; t < T; t++) {
        float lanes[32];
        for (int lane = 0; lane < 32; lane++) {
            float sum = 0.0f;
            for (int j = lane; j < hd; j += 32) {
                float pr = q[j] * keys[(size_t)t * kvd + kh * hd + j];
                sum = sum + pr;
            }
            lanes[lane] = sum;
        }
        scores[t] = refo_butterfly32(lanes) * qscale;
    }
    float mx = -3.402823466e38f;
    for (int t = 0; t < T; t++) mx = fmaxf(mx, scores[t]);
    float red[128];
    for (int tid = 0; tid < 128; tid++) {
        float total = 0.0f;
        for (int t = tid; t < T; t += 128) {
            float e = uqo_expf(scores[t] - mx);
            scores[t] = e;
            total = total + e;
        }
        red[tid] = total;
    }
    for (int d = 64; d; d >>= 1)
        for (int tid = 0; tid < d; tid++) red[tid] = red[tid] + red[tid + d];
    const float total = red[0];
    for (int t = 0; t < T; t++) scores[t] = scores[t] / total;
    for (int i = 0; i < hd; i++) {
        float sum = 0.0f;
        for (int t = 0; t < T; t++) {
            float pr = scores[t] * values[(size_t)t * kvd + kh * hd + i];
            sum = sum + pr;
        }
        out[i] = sum;
    }
    free(scores);
}

static float refo_kv(const uqo_refo* s, float v) {
    return s->kv_fp16 ? uqo_half(uqo_f16_rne(v)) : v;
}

int uqo_refo_decode(uqo_refo* s, uint32_t token, int pos, uint32_t* next, float* logits) {
    const uqo_qwen2* m = &s->m;
    if (pos < 0 || pos >= m->max_seq || (int64_t)token >= m->vocab) return -2;
    const int D = m->dim, H = m->hidden, hd = m->head_dim, kvd = m->kv_heads * hd, half = hd / 2;
    const int group = m->heads / m->kv_heads;
    float *x = malloc(sizeof(float) * D), *tmp = calloc(D, sizeof(float)), *xn = malloc(sizeof(float) * D);
    float *q = malloc(sizeof(float) * D), *k = malloc(sizeof(float) * kvd), *v = malloc(sizeof(float) * kvd);
    float *att = malloc(sizeof(float) * D), *gate = malloc(sizeof(float) * H);
    float *xs = malloc(sizeof(float) * (H / 32));
    int8_t* xq = malloc(H);
    int rc = 0;
    embed(m, token, x);
    const float* trig = s->trig + (size_t)pos * hd;
    for (int l = 0; l < m->layers; l++) {
        const uqo_layer* L = &m->layer[l];
        float* kc = s->keys + ((size_t)l * m->max_seq) * kvd;
        float* vc = s->values + ((size_t)l * m->max_seq) * kvd;
        uqo_refo_resnorm(x, tmp, L->attn_norm, xn, D, m->eps, l > 0);
        uqo_quant_act(xn, D, xs, xq);
        refo_dotrows(L->wq, D, D, xs, xq, q);
        refo_dotrows(L->wk, D, kvd, xs, xq, k);
        refo_dotrows(L->wv, D, kvd, xs, xq, v);
        /* rope_bias: q and k rotated after the bias add, v biased */
        for (int h = 0; h < m->heads; h++)
            for (int j = 0; j < half; j++) {
                const int a = h * hd + j, b = a + half;
                const float cs = trig[j], sn = trig[half + j];
                const float u = L->bq ? q[a] + L->bq[a] : q[a], w = L->bq ? q[b] + L->bq[b] : q[b];
                const float p0 = u * cs, p1 = w * sn, p2 = u * sn, p3 = w * cs;
                q[a] = p0 - p1;
                q[b] = p2 + p3;
            }
        for (int h = 0; h < m->kv_heads; h++)
            for (int j = 0; j < half; j++) {
                const int a = h * hd + j, b = a + half;
                const float cs = trig[j], sn = trig[half + j];
                const float u = L->bk ? k[a] + L->bk[a] : k[a], w = L->bk ? k[b] + L->bk[b] : k[b];
                const float p0 = u * cs, p1 = w * sn, p2 = u * sn, p3 = w * cs;
                kc[(size_t)pos * kvd + a] = refo_kv(s, p0 - p1);
                kc[(size_t)pos * kvd + b] = refo_kv(s, p2 + p3);
            }
        for (int i = 0; i < kvd; i++) vc[(size_t)pos * kvd + i] = refo_kv(s, L->bv ? v[i] + L->bv[i] : v[i]);
        #pragma omp parallel for schedule(static)
        for (int h = 0; h < m->heads; h++)
            uqo_refo_attention_head(q + h * hd, kc, vc, pos, kvd, h / group, hd, att + h * hd);
        uqo_quant_act(att, D, xs, xq);
        refo_linear(L->wo, D, D, xs, xq, tmp);
        uqo_refo_resnorm(x, tmp, L->ffn_norm, xn, D, m->eps, 1);
        uqo_quant_act(xn, D, xs, xq);
        #pragma omp parallel for schedule(static)
        for (int r = 0; r < H; r++) {
            const int64_t rb = (int64_t)(D / 32) * 34;
            const float g = uqo_refo_dotrow(L->wg + r * rb, xs, xq, D / 32);
            const float u = uqo_refo_dotrow(L->wu + r * rb, xs, xq, D / 32);
            const float e = uqo_expf(-g);
            const float den = 1.0f + e;
            const float sg = g / den;
            gate[r] = sg * u;
        }
        uqo_quant_act(gate, H, xs, xq);
        refo_linear(L->wd, H, D, xs, xq, tmp);
        if (!all_finite(tmp, D)) { rc = -3; goto done; }
    }
    {
        uqo_refo_resnorm(x, tmp, m->output_norm, xn, D, m->eps, 1);
        uqo_quant_act(xn, D, xs, xq);
        float* lg = logits ? logits : (float*)malloc(sizeof(float) * (size_t)m->vocab);
        refo_linear(m->output, D, m->vocab, xs, xq, lg);
        int bad = 0;
        const int id = uqo_greedy(lg, m->vocab, &bad);
        if (next) *next = (uint32_t)id;
        if (!logits) free(lg);
        rc = bad ? -1 : 0;
    }
done:
    free(x); free(tmp); free(xn); free(q); free(k); free(v); free(att); free(gate); free(xs); free(xq);
    return rc;
}
