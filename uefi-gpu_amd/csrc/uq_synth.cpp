// Seeded synthetic weights and inputs for the quantized-matmul path.
//
// Generator: SplitMix64-seeded PCG32 (XSH-RR 64/32). Every row of a tensor has
// its own PCG32 stream, so rows are generated in parallel and the bytes do not
// depend on the thread count:
//   s = seed + 0x9E3779B97F4A7C15 * (row + 1)
//   initstate = splitmix64_next(&s); initseq = splitmix64_next(&s)
//   pcg32_srandom(initstate, initseq)
// Bounded integers use rejection (threshold = 2^32 mod range), normals use
// Box-Muller (cos branch, double precision), fp16 values round to nearest even.
//
// Draw order inside one block (the byte layouts are GGUF's):
//   Q8_0: d = fp16(lognormal), then 32 x q uniform in [-127,127]
//   Q4_K: d, dmin (lognormal), 8 scales, 8 mins uniform in [0,63], 256 q in [0,15]
//   Q3_K: 256 q3 uniform in [0,7] (low 2 bits -> qs, bit 2 -> hmask),
//         16 scales uniform in [0,63], d (lognormal)
// lognormal = exp(ln(median) + sigma * N(0,1)), median 0.01 and sigma 0.5.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>
#include <algorithm>

namespace {

inline uint64_t splitmix64_next(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Pcg32 {
    uint64_t state = 0, inc = 1;
    uint32_t next() {
        uint64_t old = state;
        state = old * 6364136223846793005ull + inc;
        uint32_t xorshifted = (uint32_t)(((old >> 18) ^ old) >> 27);
        uint32_t rot = (uint32_t)(old >> 59);
        return (xorshifted >> rot) | (xorshifted << ((32u - rot) & 31u));
    }
    void seed(uint64_t initstate, uint64_t initseq) {
        state = 0;
        inc = (initseq << 1) | 1u;
        next();
        state += initstate;
        next();
    }
    static Pcg32 row_stream(uint64_t seed, uint64_t row) {
        uint64_t s = seed + 0x9E3779B97F4A7C15ull * (row + 1);
        uint64_t a = splitmix64_next(&s), b = splitmix64_next(&s);
        Pcg32 p;
        p.seed(a, b);
        return p;
    }
    // uniform integer in [lo, hi], hi - lo < 2^32
    int64_t range(int64_t lo, int64_t hi) {
        uint64_t span = (uint64_t)(hi - lo) + 1;
        if (span >= (1ull << 32)) return lo + next();
        uint32_t r32 = (uint32_t)span, threshold = (uint32_t)(0u - r32) % r32;
        for (;;) {
            uint32_t r = next();
            if (r >= threshold) return lo + (int64_t)(r % r32);
        }
    }
    double unit_open0() { return ((double)next() + 1.0) / 4294967296.0; }  // (0, 1]
    double unit() { return (double)next() / 4294967296.0; }                // [0, 1)
    double normal() {
        double u1 = unit_open0(), u2 = unit();
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    }
};

uint16_t f16_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        float a;
        std::memcpy(&a, &ax, 4);
        return (uint16_t)(sign | (uint32_t)std::nearbyint(a * 16777216.0f));
    }
    uint32_t e = (ax >> 23) - 112u, mant = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (mant >> 13), rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

inline uint16_t lognormal_f16(Pcg32& g) {
    double z = g.normal();
    return f16_rne((float)std::exp(std::log(0.01) + 0.5 * z));
}
inline void put16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

void gen_q8_0_row(Pcg32& g, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / 32; b++) {
        uint8_t* p = out + b * 34;
        put16(p, lognormal_f16(g));
        for (int j = 0; j < 32; j++) p[2 + j] = (uint8_t)(int8_t)g.range(-127, 127);
    }
}

void gen_q4_k_row(Pcg32& g, int64_t n, uint8_t* out) {
    for (int64_t s = 0; s < n / 256; s++) {
        uint8_t* p = out + s * 144;
        put16(p, lognormal_f16(g));
        put16(p + 2, lognormal_f16(g));
        int sc[8], mn[8];
        for (int j = 0; j < 8; j++) sc[j] = (int)g.range(0, 63);
        for (int j = 0; j < 8; j++) mn[j] = (int)g.range(0, 63);
        uint8_t* q = p + 4;  // inverse of ggml get_scale_min_k4
        for (int j = 0; j < 4; j++) {
            q[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
            q[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
        }
        for (int j = 4; j < 8; j++) q[j + 4] = (uint8_t)((sc[j] & 0xF) | ((mn[j] & 0xF) << 4));
        uint8_t* qs = p + 16;
        std::memset(qs, 0, 128);
        for (int i = 0; i < 256; i++) {
            int v = (int)g.range(0, 15), j = i >> 6, h = (i >> 5) & 1, l = i & 31;
            qs[32 * j + l] |= (uint8_t)(v << (4 * h));
        }
    }
}

void gen_q3_k_row(Pcg32& g, int64_t n, uint8_t* out) {
    for (int64_t s = 0; s < n / 256; s++) {
        uint8_t* p = out + s * 110;
        uint8_t *hm = p, *qs = p + 32, *sc = p + 96;
        std::memset(p, 0, 110);
        for (int i = 0; i < 256; i++) {
            int v = (int)g.range(0, 7);
            int nn = i >> 7, j = (i >> 5) & 3, h = (i >> 4) & 1, l = i & 15;
            qs[32 * nn + 16 * h + l] |= (uint8_t)((v & 3) << (2 * j));
            if (v & 4) hm[16 * h + l] |= (uint8_t)(1u << (4 * nn + j));
        }
        int scl[16];
        for (int k = 0; k < 16; k++) scl[k] = (int)g.range(0, 63);
        for (int k = 0; k < 16; k++) {  // inverse of the ggml 12-byte 6-bit packing
            if (k < 8) sc[k] |= (uint8_t)(scl[k] & 0xF);
            else sc[k - 8] |= (uint8_t)((scl[k] & 0xF) << 4);
            sc[8 + (k & 3)] |= (uint8_t)(((scl[k] >> 4) & 3) << (2 * (k >> 2)));
        }
        put16(p + 108, lognormal_f16(g));
    }
}

// The fp32-activation reader's kinds: uniform random code bytes with each
// block's fp16 scale field lognormal (median 0.01, sigma 0.5); F32/BF16 rows
// are 0.05 * N(0,1) (BF16 rounded to nearest even from the f32).
void gen_frontier_row(Pcg32& g, uint32_t kind, int64_t n, uint8_t* out, int64_t rb) {
    if (kind == 0 || kind == 30) {
        for (int64_t i = 0; i < n; i++) {
            const float v = (float)(0.05 * g.normal());
            uint32_t b;
            std::memcpy(&b, &v, 4);
            if (kind == 0) std::memcpy(out + 4 * i, &b, 4);
            else put16(out + 2 * i, (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16));
        }
        return;
    }
    for (int64_t i = 0; i < rb; i++) out[i] = (uint8_t)g.next();
    int64_t block, size, off;
    switch (kind) {
    case 14: block = 256; size = 210; off = 208; break;
    case 18: block = 256; size = 98; off = 0; break;
    case 20: block = 32; size = 18; off = 0; break;
    default: block = 256; size = 136; off = 0; break;  // 23
    }
    for (int64_t b = 0; b < n / block; b++) put16(out + b * size + off, lognormal_f16(g));
}

template <class F>
void parallel_rows(int64_t rows, F&& f) {
    unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (rows < 64 || hw == 1) {
        for (int64_t r = 0; r < rows; r++) f(r);
        return;
    }
    std::vector<std::thread> pool;
    int64_t chunk = (rows + hw - 1) / hw;
    for (unsigned t = 0; t < hw; t++) {
        int64_t lo = t * chunk, hi = std::min(rows, lo + chunk);
        if (lo >= hi) break;
        pool.emplace_back([lo, hi, &f] { for (int64_t r = lo; r < hi; r++) f(r); });
    }
    for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

// GGUF-layout quantized rows (kind: 8 Q8_0, 11 Q3_K, 12 Q4_K, and the
// fp32-activation reader's 0 F32, 14 Q6_K, 18 IQ3_XXS, 20 IQ4_NL, 23 IQ4_XS,
// 30 BF16); out holds
// rows * row_bytes(kind, n). Returns 0, or -1 for an unknown kind / bad n.
int uq_synth_quant(uint32_t kind, uint64_t seed, int64_t rows, int64_t n, uint8_t* out) {
    int64_t rb;
    if (kind == 8 && n > 0 && n % 32 == 0) rb = n / 32 * 34;
    else if (kind == 12 && n > 0 && n % 256 == 0) rb = n / 256 * 144;
    else if (kind == 11 && n > 0 && n % 256 == 0) rb = n / 256 * 110;
    else if (kind == 14 && n > 0 && n % 256 == 0) rb = n / 256 * 210;
    else if (kind == 18 && n > 0 && n % 256 == 0) rb = n / 256 * 98;
    else if (kind == 20 && n > 0 && n % 32 == 0) rb = n / 32 * 18;
    else if (kind == 23 && n > 0 && n % 256 == 0) rb = n / 256 * 136;
    else if (kind == 0 && n > 0) rb = n * 4;
    else if (kind == 30 && n > 0) rb = n * 2;
    else return -1;
    if (rows <= 0 || !out) return -1;
    parallel_rows(rows, [&](int64_t r) {
        Pcg32 g = Pcg32::row_stream(seed, (uint64_t)r);
        if (kind != 8 && kind != 11 && kind != 12) gen_frontier_row(g, kind, n, out + r * rb, rb);
        else if (kind == 8) gen_q8_0_row(g, n, out + r * rb);
        else if (kind == 12) gen_q4_k_row(g, n, out + r * rb);
        else gen_q3_k_row(g, n, out + r * rb);
    });
    return 0;
}

// n values mean + std * N(0,1), as float32 from stream row 0.
int uq_synth_normal(uint64_t seed, int64_t n, float mean, float stddev, float* out) {
    if (n < 0 || (n && !out)) return -1;
    Pcg32 g = Pcg32::row_stream(seed, 0);
    for (int64_t i = 0; i < n; i++) out[i] = (float)((double)mean + (double)stddev * g.normal());
    return 0;
}

// n token ids uniform in [0, vocab), stream row 0.
int uq_synth_tokens(uint64_t seed, int64_t n, uint32_t vocab, uint32_t* out) {
    if (n < 0 || vocab == 0 || (n && !out)) return -1;
    Pcg32 g = Pcg32::row_stream(seed, 0);
    for (int64_t i = 0; i < n; i++) out[i] = (uint32_t)g.range(0, (int64_t)vocab - 1);
    return 0;
}

}  // extern "C"
