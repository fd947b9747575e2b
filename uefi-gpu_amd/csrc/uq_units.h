// Per-kind matvec work units shared by the generic matvec and the fused
// decode-step kernels. A unit is the slice of one row that one lane consumes
// per step: Q8_0 16 values (one 16-byte load), Q4_K 64 values (one 32-byte qs
// pair + the superblock header), Q3_K 128 values (half a superblock).
// load_w(w, row, nu, u) issues the unit's weight loads and nothing else;
// dot(W, X, u) returns the unit's double contribution to the row's dot;
// term() = dot(load_w()). Kernels issue every unit's load_w of a row before
// the first dot, so a row costs one memory round trip.
#pragma once
#include "uq_device.h"

namespace uq {

struct WArgs {
    const int8_t* qs;
    const uint16_t* d;
    const uint8_t* sc;
};

// Q8_0 unit: half a block (16 int8 = one 16-byte load). Lanes of a row group
// read consecutive 16-byte pieces, so one wave instruction covers a contiguous
// run of the row; weights are streamed with non-temporal loads. The two halves
// of a block contribute exact double terms c_half * (dw*dx) whose sum equals
// the block's c * (dw*dx) exactly.
struct Q8 {
    static constexpr int UNIT = 16;
    struct X { int4 a; float s; };
    static UQ_DEV void load_x(X& x, const int8_t* xq, const float* xs, int u) {
        x.a = *(const int4*)(xq + (size_t)u * 16);
        x.s = xs[u >> 1];
    }
    struct W { int4 q; uint16_t d; };
    // row base pointers, formed once per row (nu is even: K % 32 == 0)
    struct R { const int8_t* q; const uint16_t* d; };
    static UQ_DEV R row_ptr(const WArgs& w, int64_t row, int64_t nu) {
        return R{w.qs + row * nu * 16, w.d + row * (nu >> 1)};
    }
    // weight part of unit u of the row, loadable before the activations are known
    static UQ_DEV W load_u(const R& r, int u) { return W{uq_ntload16(r.q + (int64_t)u * 16), r.d[u >> 1]}; }
    static UQ_DEV W load_w(const WArgs& w, int64_t row, int64_t nu, int u) { return load_u(row_ptr(w, row, nu), u); }
    static UQ_DEV double dot(const W& wv, const X& x, int = 0) {
        int c = uq_dot4(wv.q.x, x.a.x, 0);
        c = uq_dot4(wv.q.y, x.a.y, c);
        c = uq_dot4(wv.q.z, x.a.z, c);
        c = uq_dot4(wv.q.w, x.a.w, c);
        const float s = uq_half(wv.d) * x.s;
        return (double)c * (double)s;
    }
    static UQ_DEV double term(const WArgs& w, int64_t row, int64_t nu, int u, const X& x) {
        return dot(load_w(w, row, nu, u), x);
    }
};

// Q4_K unit: pair j of a superblock = 32 bytes of qs holding sub-blocks 2j (low
// nibbles) and 2j+1 (high nibbles). ggml value = d*sc*q - dmin*m per sub-block.
// Planes (repacked at upload, byte-verified): the nibble plane holds, per row,
// the first 16 bytes of every unit and then their second 16 bytes, so each of
// a unit's two non-temporal 16-byte loads is contiguous across the row's lanes;
// scm[sb][4 pairs] = one word per unit: scale(2j) | scale(2j+1) << 8 |
// min(2j) << 16 | min(2j+1) << 24 (the 6-bit fields unpacked to bytes);
// dm[sb] = d | dmin (fp16 pair). scm and dm go through the cache (the
// four lanes of a superblock share them). The activation scales and sums of a
// unit (the sums feed the min term) are formed once when it is loaded.
struct Q4K {
    static constexpr int UNIT = 64;
    struct X { int4 a0, a1, b0, b1; double s0, s1; int xl, xh; };
    static UQ_DEV int sum16(const int4& v, int c) {
        const int ones = 0x01010101;
        c = uq_dot4(ones, v.x, c); c = uq_dot4(ones, v.y, c);
        c = uq_dot4(ones, v.z, c); return uq_dot4(ones, v.w, c);
    }
    static UQ_DEV void load_x(X& x, const int8_t* xq, const float* xs, int u) {
        const int4* p = (const int4*)(xq + (size_t)u * 64);
        x.a0 = p[0]; x.a1 = p[1]; x.b0 = p[2]; x.b1 = p[3];
        x.s0 = (double)xs[2 * u];
        x.s1 = (double)xs[2 * u + 1];
        x.xl = sum16(x.a1, sum16(x.a0, 0));
        x.xh = sum16(x.b1, sum16(x.b0, 0));
    }
    // the staged 16-value sum of group g of the row (used as is)
    static UQ_DEV int stage16(int, int sum) { return sum; }
    // from an activation staged with its 16-value sums s16 (LDS)
    static UQ_DEV void load_x_pre(X& x, const int8_t* xq, const float* xs, const int* s16, int u) {
        const int4* p = (const int4*)(xq + (size_t)u * 64);
        x.a0 = p[0]; x.a1 = p[1]; x.b0 = p[2]; x.b1 = p[3];
        x.s0 = (double)xs[2 * u];
        x.s1 = (double)xs[2 * u + 1];
        x.xl = s16[4 * u] + s16[4 * u + 1];
        x.xh = s16[4 * u + 2] + s16[4 * u + 3];
    }
    static UQ_DEV int lo4(int w) { return w & 0x0F0F0F0F; }
    static UQ_DEV int hi4(int w) { return (int)(((unsigned)w >> 4) & 0x0F0F0F0Fu); }
    struct W { int4 q0, q1; uint32_t scm, dm; };
    // row base pointers (nu = 4 * superblocks per row): the nibble plane row,
    // its second halves nu*16 bytes on, one scm word per unit, one dm word per
    // superblock
    struct R { const uint8_t* q; int64_t half; const uint32_t* scm; const uint32_t* dm; };
    static UQ_DEV R row_ptr(const WArgs& w, int64_t row, int64_t nu) {
        return R{(const uint8_t*)w.qs + row * nu * 32, nu * 16, (const uint32_t*)w.sc + row * nu,
                 (const uint32_t*)w.d + row * (nu >> 2)};
    }
    static UQ_DEV W load_u(const R& r, int u) {
        const uint8_t* q = r.q + (int64_t)u * 16;
        return W{uq_ntload16(q), uq_ntload16(q + r.half), r.scm[u], r.dm[u >> 2]};
    }
    static UQ_DEV W load_w(const WArgs& w, int64_t row, int64_t nu, int u) { return load_u(row_ptr(w, row, nu), u); }
    static UQ_DEV double dot(const W& wv, const X& x, int = 0) {
        const int4 q0 = wv.q0, q1 = wv.q1;
        int il = 0, ih = 0;
        il = uq_dot4(lo4(q0.x), x.a0.x, il); il = uq_dot4(lo4(q0.y), x.a0.y, il);
        il = uq_dot4(lo4(q0.z), x.a0.z, il); il = uq_dot4(lo4(q0.w), x.a0.w, il);
        il = uq_dot4(lo4(q1.x), x.a1.x, il); il = uq_dot4(lo4(q1.y), x.a1.y, il);
        il = uq_dot4(lo4(q1.z), x.a1.z, il); il = uq_dot4(lo4(q1.w), x.a1.w, il);
        ih = uq_dot4(hi4(q0.x), x.b0.x, ih); ih = uq_dot4(hi4(q0.y), x.b0.y, ih);
        ih = uq_dot4(hi4(q0.z), x.b0.z, ih); ih = uq_dot4(hi4(q0.w), x.b0.w, ih);
        ih = uq_dot4(hi4(q1.x), x.b1.x, ih); ih = uq_dot4(hi4(q1.y), x.b1.y, ih);
        ih = uq_dot4(hi4(q1.z), x.b1.z, ih); ih = uq_dot4(hi4(q1.w), x.b1.w, ih);
        // d*sc and dmin*m are exact in f32 (11-bit x 6-bit), so (d*sc)*isum ==
        // d*(sc*isum) with an exact integer inner product; same for the min term
        const double dd = (double)uq_half((uint16_t)(wv.dm & 0xffff));
        const double dm = (double)uq_half((uint16_t)(wv.dm >> 16));
        const int sc0 = (int)(wv.scm & 0xff), sc1 = (int)((wv.scm >> 8) & 0xff);
        const int m0 = (int)((wv.scm >> 16) & 0xff), m1 = (int)(wv.scm >> 24);
        // 24-bit multiplies (full rate): |sc|, |m| <= 63, |il| <= 61,440, |xl| <= 4,064
        const double t0 = x.s0 * (dd * (double)uq_mul24(sc0, il) - dm * (double)uq_mul24(m0, x.xl));
        const double t1 = x.s1 * (dd * (double)uq_mul24(sc1, ih) - dm * (double)uq_mul24(m1, x.xh));
        return t0 + t1;
    }
    static UQ_DEV double term(const WArgs& w, int64_t row, int64_t nu, int u, const X& x) {
        return dot(load_w(w, row, nu, u), x, u);
    }
    // dot against an activation staged in LDS with its 16-value sums
    static UQ_DEV double dot_lds(const W& wv, const int8_t* lx, const float* lxs, const int* ls16, int u) {
        X x;
        load_x_pre(x, lx, lxs, ls16, u);
        return dot(wv, x, u);
    }
    // ggml get_scale_min_k4: 12 packed bytes b -> scale and min of sub-block k
    static UQ_HD void scale_min_k4(const uint8_t* b, int k, int& sc, int& m) {
        if (k < 4) {
            sc = b[k] & 63;
            m = b[k + 4] & 63;
        } else {
            sc = (b[k + 4] & 0xF) | ((b[k - 4] >> 6) << 4);
            m = (b[k + 4] >> 4) | ((b[k] >> 6) << 4);
        }
    }
};

// Q3_K unit: a quarter of a superblock = 64 consecutive values = activation
// blocks 2u and 2u+1 = the four 16-value sub-blocks 4p..4p+3 of the GGUF
// superblock (p = u mod 4), each with its 6-bit scale s (factor s - 32). GGUF
// value = low2 - 4*(1 - hbit) = v3 - 4 with v3 = low2 | hbit << 2 in 0..7.
// Planes (repacked at upload, byte-verified), per unit:
//   q[u][16]: words A_t, t = 0..3; byte b of A_t holds value 16c + 4t + b of
//             sub-block c as: bits 0-2 v3 (c = 0), bit 3 hbit (c = 1), bits
//             4-6 v3 (c = 2), bit 7 hbit (c = 3);
//   p[u][16]: words B_0, B_1 with the low2 of sub-blocks 1 and 3: byte b of
//             B_a holds t = 2a at bits 0-1 (c = 1) and 4-5 (c = 3), t = 2a+1 at
//             bits 2-3 and 6-7; then the four s - 32 as signed bytes; then the
//             superblock's fp16 d (upper half 0).
// Sub-blocks 0 and 2 assemble with one AND per word (2 at 16x scale), 1 and 3
// with one AND-OR of B and the once-shifted A (3 at 16x scale). Each lane's
// loads are two 16-byte pieces per unit, each contiguous across the lanes of
// a row (a load instruction costs about the same for 2, 12 or 16 bytes per
// lane, so d rides in the second piece: 128 B per superblock, 16% over GGUF).
struct Q3K {
    static constexpr int UNIT = 64;
    // v: the unit's 64 activations by sub-block; s0, s1: the two block
    // scales; c: per sub-block c the start of its dot, -4 * GS(c) * (sum of
    // its 16 activations), GS = 1 for sub-blocks 0-1 and 16 for 2-3
    struct X { int4 v[4]; double s0, s1; int4 c; };
    static UQ_DEV int gs_corr(int c, int sum) { return uq_mul24(sum, c >= 2 ? -64 : -4); }
    // the staged 16-value sum of group g of the row, as the dot's start
    static UQ_DEV int stage16(int g, int sum) { return gs_corr(g & 3, sum); }
    static UQ_DEV int sum16(const int4& v) {
        const int ones = 0x01010101;
        int c = uq_dot4(ones, v.x, 0);
        c = uq_dot4(ones, v.y, c);
        c = uq_dot4(ones, v.z, c);
        return uq_dot4(ones, v.w, c);
    }
    static UQ_DEV void load_x(X& x, const int8_t* xq, const float* xs, int u) {
        const int4* p = (const int4*)(xq + (size_t)u * 64);
#pragma unroll
        for (int k = 0; k < 4; k++) x.v[k] = p[k];
        x.s0 = (double)xs[2 * u];
        x.s1 = (double)xs[2 * u + 1];
        x.c = make_int4(gs_corr(0, sum16(x.v[0])), gs_corr(1, sum16(x.v[1])), gs_corr(2, sum16(x.v[2])),
                        gs_corr(3, sum16(x.v[3])));
    }
    // from an activation staged with stage16's starts (LDS)
    static UQ_DEV void load_x_pre(X& x, const int8_t* xq, const float* xs, const int* s16, int u) {
        const int4* p = (const int4*)(xq + (size_t)u * 64);
#pragma unroll
        for (int k = 0; k < 4; k++) x.v[k] = p[k];
        x.s0 = (double)xs[2 * u];
        x.s1 = (double)xs[2 * u + 1];
        x.c = *(const int4*)(s16 + 4 * u);
    }
    struct W { int4 a; int4 p; };
    // row base pointers (nu = 4 * superblocks per row)
    struct R { const uint8_t* a; const uint8_t* p; };
    static UQ_DEV R row_ptr(const WArgs& w, int64_t row, int64_t nu) {
        return R{(const uint8_t*)w.qs + row * nu * 16, w.sc + row * nu * 16};
    }
    static UQ_DEV W load_u(const R& r, int u) {
        return W{uq_ntload16(r.a + (int64_t)u * 16), uq_ntload16(r.p + (int64_t)u * 16)};
    }
    static UQ_DEV W load_w(const WArgs& w, int64_t row, int64_t nu, int u) { return load_u(row_ptr(w, row, nu), u); }
    static UQ_DEV int lane4(const int4& v, int t) { return t == 0 ? v.x : (t == 1 ? v.y : (t == 2 ? v.z : v.w)); }
    // The unit's dot: per word t the four sub-block dwords, then the scales.
    // T0 = s0*D0 + s1*D1 (GS 1) and T1 = s2*D2 + s3*D3 (GS 16) are exact
    // integers (|D| <= 16 * 4 * 16 * 127, |s| <= 32); d*(s-32) is exact in
    // f32 (11-bit x 6-bit), so the blocks' sums of (d*s)*D equal d*T, and
    // d * xs is exact in double.
    // The four sub-block dwords of word t (values 4t..4t+3 of each
    // sub-block as int8 lanes, v3 scaled by GS = 1, 1, 16, 16) from A_t and
    // the B word pair holding t.
    static UQ_HD void words(uint32_t A, uint32_t Bw, int t, int* w) {
        const uint32_t B = (t & 1) ? Bw >> 2 : Bw;
        const uint32_t As = A >> 1;
        w[0] = (int)(A & 0x07070707u);
        w[1] = (int)((B & 0x03030303u) | (As & 0x04040404u));
        w[2] = (int)(A & 0x70707070u);
        w[3] = (int)((B & 0x30303030u) | (As & 0x40404040u));
    }
    static UQ_DEV double dot_v(const W& wv, const int4* xv, const int4& c, double xs0, double xs1) {
        int D0 = c.x, D1 = c.y, D2 = c.z, D3 = c.w;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            int w[4];
            words((uint32_t)lane4(wv.a, t), (uint32_t)(t < 2 ? wv.p.x : wv.p.y), t, w);
            D0 = uq_dot4(w[0], lane4(xv[0], t), D0);
            D1 = uq_dot4(w[1], lane4(xv[1], t), D1);
            D2 = uq_dot4(w[2], lane4(xv[2], t), D2);
            D3 = uq_dot4(w[3], lane4(xv[3], t), D3);
        }
        const int s = wv.p.z;
        const int s0 = (int)(int8_t)s, s1 = (int)(int8_t)(s >> 8), s2 = (int)(int8_t)(s >> 16), s3 = s >> 24;
        const int T0 = uq_mul24(s0, D0) + uq_mul24(s1, D1);
        const int T1 = uq_mul24(s2, D2) + uq_mul24(s3, D3);
        const double dd = (double)uq_half((uint16_t)wv.p.w);
        return (dd * xs0) * (double)T0 + (dd * (xs1 * (1.0 / 16))) * (double)T1;
    }
    static UQ_DEV double dot(const W& wv, const X& x, int = 0) { return dot_v(wv, x.v, x.c, x.s0, x.s1); }
    static UQ_DEV double term(const WArgs& w, int64_t row, int64_t nu, int u, const X& x) {
        return dot(load_w(w, row, nu, u), x, u);
    }
    // dot against an activation staged in LDS with stage16's starts
    static UQ_DEV double dot_lds(const W& wv, const int8_t* lx, const float* lxs, const int* ls16, int u) {
        const int4* p = (const int4*)(lx + (size_t)u * 64);
        const int4 xv[4] = {p[0], p[1], p[2], p[3]};
        const int4 c = *(const int4*)(ls16 + 4 * u);
        const float2 xs = *(const float2*)(lxs + 2 * u);
        return dot_v(wv, xv, c, (double)xs.x, (double)xs.y);
    }
    // ggml Q3_K 6-bit scale k (0..15) of the 12 packed bytes b
    static UQ_HD int scale6_k(const uint8_t* b, int k) {
        const int low = k < 8 ? (b[k] & 0xF) : (b[k - 8] >> 4);
        const int high = (b[8 + (k & 3)] >> (2 * (k >> 2))) & 3;
        return low | (high << 4);
    }
    // GGUF superblock g (hmask 32, qs 64, scales 12, d 2): low 2 bits and
    // high bit of value i (0..255)
    static UQ_HD int gguf_low2(const uint8_t* g, int i) {
        const int n = i >> 7, j = (i >> 5) & 3, l = i & 31;
        return (g[32 + 32 * n + l] >> (2 * j)) & 3;
    }
    static UQ_HD int gguf_hbit(const uint8_t* g, int i) {
        const int n = i >> 7, j = (i >> 5) & 3, l = i & 31;
        return (g[l] >> (4 * n + j)) & 1;
    }
    // Unit p's plane words from GGUF superblock g: A[4], P[4]
    static UQ_HD void pack_unit(const uint8_t* g, int p, uint32_t* A, uint32_t* P) {
        for (int t = 0; t < 4; t++) {
            uint32_t a = 0;
            for (int b = 0; b < 4; b++) {
                const int i = 64 * p + 4 * t + b;  // + 16c
                const uint32_t v0 = gguf_low2(g, i) | gguf_hbit(g, i) << 2;
                const uint32_t v2 = gguf_low2(g, i + 32) | gguf_hbit(g, i + 32) << 2;
                const uint32_t byte = v0 | (uint32_t)gguf_hbit(g, i + 16) << 3 | v2 << 4 |
                                      (uint32_t)gguf_hbit(g, i + 48) << 7;
                a |= byte << (8 * b);
            }
            A[t] = a;
        }
        for (int h = 0; h < 2; h++) {
            uint32_t w = 0;
            for (int b = 0; b < 4; b++) {
                const int ie = 64 * p + 4 * (2 * h) + b, io = ie + 4;
                const uint32_t byte = gguf_low2(g, ie + 16) | gguf_low2(g, ie + 48) << 4 |
                                      gguf_low2(g, io + 16) << 2 | gguf_low2(g, io + 48) << 6;
                w |= byte << (8 * b);
            }
            P[h] = w;
        }
        uint32_t s = 0;
        for (int c = 0; c < 4; c++) s |= (uint32_t)(uint8_t)(int8_t)(scale6_k(g + 96, 4 * p + c) - 32) << (8 * c);
        P[2] = s;
        P[3] = (uint32_t)g[108] | (uint32_t)g[109] << 8;
    }
    // low 2 bits and high bit of value 16c + 4t + b of a unit from its plane words
    static UQ_HD void unit_parts(const uint32_t* A, const uint32_t* P, int c, int t, int b, int& low2, int& hbit) {
        const uint32_t a = (A[t] >> (8 * b)) & 0xff;
        const uint32_t bb = ((P[t >> 1] >> (8 * b)) & 0xff) >> (2 * (t & 1));
        if (c == 0) { low2 = a & 3; hbit = (a >> 2) & 1; }
        else if (c == 2) { low2 = (a >> 4) & 3; hbit = (a >> 6) & 1; }
        else if (c == 1) { low2 = bb & 3; hbit = (a >> 3) & 1; }
        else { low2 = (bb >> 4) & 3; hbit = a >> 7; }
    }
};

// ---------------------------------------------------------------- row-block layout
// lm_head-sized Q3_K weights are stored in row blocks in which one lane owns
// one whole superblock and moves it as 16-byte pieces only. A block
// has LB lane slots (1 to 4 whole waves) holding RB = LB / S rows of S = K / 256
// superblocks (slot j = row-in-block * S + superblock; slots from RB * S on
// are padding); piece k of slot j sits at block * LB * P * 16 + k * LB * 16 +
// j * 16, so one load instruction of a wave reads 64 consecutive pieces, a
// kilobyte of whole cache lines. Q3KSB, P = 7: pieces 0..3 the A words of
// the four 64-value units (the Q3K unit words), piece 4 the B words of units
// 0 and 1, piece 5 those of units 2 and 3, piece 6 the sixteen scales - 32
// as signed 6-bit fields (unit u's four at bits 24u + 6c of the first 96
// bits) and d in the low half of the last word: 112 bytes for GGUF's 110.
// (The same layout for Q4_K, its 144-byte superblock verbatim in 9 pieces,
// measured 70-71% of 8 TB/s on lm_head against 76-77% for the Q4K unit
// planes, and 74-75% with the dots removed: its access pattern, not its
// arithmetic, bounds it, so Q4_K keeps the unit planes.)
struct SbGeom {
    int S = 0, LB = 0, RB = 0;  // superblocks per row, lane slots and rows per block
    int64_t blocks = 0;         // row blocks (the last one may hold padding rows)
};
// The block of 64, 128, 192 or 256 slots with the smallest share of idle
// slots, the smaller block on a tie (S <= 64; else no row-block layout). At
// K = 1536 (S = 6) that is 192 slots, 32 rows and none idle, where 64 slots
// would leave 4 of every 64 idle and move 6.7% more bytes.
inline SbGeom sb_geom(int64_t n, int64_t m) {
    SbGeom g;
    if (n % 256 || n / 256 > 64 || m <= 0) return g;
    g.S = (int)(n / 256);
    for (int lb = 64; lb <= 256; lb += 64) {
        const int rb = lb / g.S;
        // idle share (lb - rb S) / lb below the best one's, cross-multiplied
        if (rb >= 1 && (!g.LB || (int64_t)(lb - rb * g.S) * g.LB < (int64_t)(g.LB - g.RB * g.S) * lb)) {
            g.LB = lb;
            g.RB = rb;
        }
    }
    g.blocks = (m + g.RB - 1) / g.RB;
    return g;
}
// Byte offset of piece k of superblock s of row r.
UQ_HD int64_t sb_piece(int64_t r, int s, int k, int S, int LB, int RB, int P) {
    const int64_t b = r / RB;
    const int j = (int)(r - b * RB) * S + s;
    return ((b * P + k) * LB + j) * 16;
}

struct Q3KSB {
    static constexpr int P = 7;
    // the eight Q3K unit words A[u][4], B[u][2], the scales - 32 as signed
    // bytes S[u] and d, into the seven pieces (28 words)
    static UQ_HD void pack(const uint32_t A[4][4], const uint32_t Pw[4][4], uint32_t* w) {
        for (int u = 0; u < 4; u++)
            for (int t = 0; t < 4; t++) w[4 * u + t] = A[u][t];
        for (int u = 0; u < 4; u++) {
            w[16 + 2 * u] = Pw[u][0];
            w[17 + 2 * u] = Pw[u][1];
        }
        uint32_t f[3] = {0, 0, 0};
        for (int u = 0; u < 4; u++)
            for (int c = 0; c < 4; c++) {
                const uint32_t v = (Pw[u][2] >> (8 * c)) & 63;  // low 6 bits of the signed byte
                const int bit = 24 * u + 6 * c;
                f[bit >> 5] |= v << (bit & 31);
                if ((bit & 31) > 26) f[(bit >> 5) + 1] |= v >> (32 - (bit & 31));
            }
        w[24] = f[0];
        w[25] = f[1];
        w[26] = f[2];
        w[27] = Pw[0][3] & 0xffff;
    }
    // unit u's 24-bit scale window (four signed 6-bit fields at 6c)
    static UQ_HD uint32_t scale_window(uint32_t f0, uint32_t f1, uint32_t f2, int u) {
        const uint64_t lo = (uint64_t)f0 | (uint64_t)f1 << 32, hi = (uint64_t)f1 | (uint64_t)f2 << 32;
        return u == 0 ? f0 : u == 1 ? (uint32_t)(lo >> 24) : u == 2 ? (uint32_t)(hi >> 16) : f2 >> 8;
    }
    static UQ_HD int scale_field(uint32_t win, int c) { return (int)(win << (26 - 6 * c)) >> 26; }
    // the inverse of pack: unit words with P[u][2] the signed scale bytes and P[u][3] = d
    static UQ_HD void unpack(const uint32_t* w, uint32_t A[4][4], uint32_t Pw[4][4]) {
        for (int u = 0; u < 4; u++) {
            for (int t = 0; t < 4; t++) A[u][t] = w[4 * u + t];
            Pw[u][0] = w[16 + 2 * u];
            Pw[u][1] = w[17 + 2 * u];
            const uint32_t win = scale_window(w[24], w[25], w[26], u);
            uint32_t sb = 0;
            for (int c = 0; c < 4; c++) sb |= (uint32_t)(uint8_t)(int8_t)scale_field(win, c) << (8 * c);
            Pw[u][2] = sb;
            Pw[u][3] = w[27] & 0xffff;
        }
    }
};

// Rows of this workgroup. When one pass of the grid covers every row, each
// workgroup takes an even contiguous share (one pass), so every CU streams
// the same number of rows: a CU's stream rate is its share of HBM bandwidth,
// and a CU with more rows than the others would set the kernel's duration.
// share = rows / gridDim.x comes from the host (a 64-bit division on the
// device costs hundreds of instructions ahead of the first weight load); the
// first rows % gridDim.x workgroups take one row more. Otherwise the grid
// strides over passes of RPB rows.
struct RowSpan {
    int64_t begin, end, step;
};
// Rows [begin, end) of workgroup b of g when `rows` are split evenly (share =
// rows / g, the first rows - share*g workgroups take one more).
__device__ __forceinline__ RowSpan even_span_of(int64_t rows, int64_t share, int64_t b, int64_t g) {
    const int64_t extra = rows - share * g;
    const int64_t begin = b * share + (b < extra ? b : extra);
    return RowSpan{begin, begin + share + (b < extra ? 1 : 0), share + 1};
}
__device__ __forceinline__ RowSpan even_span(int64_t rows, int64_t share) {
    return even_span_of(rows, share, blockIdx.x, gridDim.x);
}
template <int RPB>
__device__ __forceinline__ RowSpan row_span(int64_t rows, int64_t share) {
    if (rows <= (int64_t)gridDim.x * RPB) {
        RowSpan r = even_span(rows, share);
        r.step = RPB;
        return r;
    }
    return RowSpan{(int64_t)blockIdx.x * RPB, rows, (int64_t)gridDim.x * RPB};
}

// Activation units of one lane (units sub, sub+LPR, ...) kept in registers.
// Loads are issued unconditionally: a unit past the row end reads the last
// unit, and every consumer drops its term by a select on u < nu. (Zeroing
// such units here would overwrite registers with loads in flight, which
// makes the compiler wait for those loads before the weight loads go out.)
template <class KQ, int LPR, int NBL>
UQ_DEV void load_xr(typename KQ::X* xr, const int8_t* xq, const float* xs, int64_t nu, int sub) {
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + LPR * i;
        KQ::load_x(xr[i], xq, xs, u < nu ? u : (int)nu - 1);
    }
}
// This lane's share of row `row`, summed over the LPR lanes of its group: all
// units' weight loads first, then the dots (a unit past the row end loads
// the last unit and is dropped by a select).
template <class KQ, int LPR, int NBL>
UQ_DEV double row_dot(const WArgs& w, int64_t row, int64_t nu, int sub, const typename KQ::X* xr) {
    typename KQ::W wv[NBL];
    const typename KQ::R rp = KQ::row_ptr(w, row, nu);
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + LPR * i;
        wv[i] = KQ::load_u(rp, u < nu ? u : (int)nu - 1);
    }
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + LPR * i;
        const double t = KQ::dot(wv[i], xr[i], u < nu ? u : (int)nu - 1);
        acc += u < nu ? t : 0.0;
    }
    return uq_group_sum<LPR>(acc);
}

}  // namespace uq
