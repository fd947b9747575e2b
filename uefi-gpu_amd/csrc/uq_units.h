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
    static UQ_DEV void scale_min_k4(const uint8_t* b, int k, int& sc, int& m) {
        if (k < 4) {
            sc = b[k] & 63;
            m = b[k + 4] & 63;
        } else {
            sc = (b[k + 4] & 0xF) | ((b[k - 4] >> 6) << 4);
            m = (b[k + 4] >> 4) | ((b[k] >> 6) << 4);
        }
    }
};

// Q3_K unit: half n of a superblock = 128 values = 4 activation blocks j.
// Block j's 32 values use qs[32n .. 32n+31] bits 2j..2j+1 and hmask[0..31]
// bit 4n+j; value = low2 - 4*(1-hbit) = (low2 | hbit << 2) - 4; each 16
// values carry a 6-bit scale s (factor s - 32). Planes (repacked at upload,
// byte-verified): q[sb][96] = hmask | qs (non-temporal loads), sc[sb][16] =
// the sixteen (s - 32) as signed bytes, d[sb] fp16. The activation scales and
// the sums of each 16 activations (for the -4 offset) are formed once at load.
struct Q3K {
    static constexpr int UNIT = 128;
    struct X { int4 v[8]; double s[4]; int sx[8]; };
    static UQ_DEV int dot16(const int4& w, const int4& xv, int c) {
        c = uq_dot4(w.x, xv.x, c); c = uq_dot4(w.y, xv.y, c);
        c = uq_dot4(w.z, xv.z, c); return uq_dot4(w.w, xv.w, c);
    }
    static UQ_DEV void load_x(X& x, const int8_t* xq, const float* xs, int u) {
        const int4* p = (const int4*)(xq + (size_t)u * 128);
#pragma unroll
        for (int k = 0; k < 8; k++) x.v[k] = p[k];
#pragma unroll
        for (int k = 0; k < 4; k++) x.s[k] = (double)xs[4 * u + k];
        const int ones = 0x01010101;
#pragma unroll
        for (int k = 0; k < 8; k++) x.sx[k] = dot16(make_int4(ones, ones, ones, ones), x.v[k], 0);
    }
    static UQ_DEV void load_x_pre(X& x, const int8_t* xq, const float* xs, const int* s16, int u) {
        const int4* p = (const int4*)(xq + (size_t)u * 128);
#pragma unroll
        for (int k = 0; k < 8; k++) x.v[k] = p[k];
#pragma unroll
        for (int k = 0; k < 4; k++) x.s[k] = (double)xs[4 * u + k];
#pragma unroll
        for (int k = 0; k < 8; k++) x.sx[k] = s16[8 * u + k];
    }
    // The hmask plane is repacked at upload: GGUF bit 4n+j of a byte (the
    // high bit of value 128n + 32j + l, l the byte index) moves to bit
    // 2 + 2j + n for j < 3 and to bit n for j = 3, so that group j of unit n
    // assembles from one AND of the (for unit 1 once-shifted) hmask word and
    // one AND-OR with the 2-bit field, with the value scaled by GS[j] = 1, 4,
    // 16 (j = 3: one more shift each side, scale 1).
    static UQ_DEV int hpos(int b) { const int n = b >> 2, j = b & 3; return j < 3 ? 2 + 2 * j + n : n; }
    static UQ_DEV uint32_t hpack(uint32_t h) {
        uint32_t r = 0;
        for (int b = 0; b < 8; b++) r |= ((h >> b) & 0x01010101u) << hpos(b);
        return r;
    }
    static UQ_DEV uint32_t hunpack(uint32_t h) {
        uint32_t r = 0;
        for (int b = 0; b < 8; b++) r |= ((h >> hpos(b)) & 0x01010101u) << b;
        return r;
    }
    template <int j>
    static UQ_DEV uint32_t v3(uint32_t q, uint32_t hh) {
        if (j == 0) return (q & 0x03030303u) | (hh & 0x04040404u);
        if (j == 1) return (q & 0x0C0C0C0Cu) | (hh & 0x10101010u);
        if (j == 2) return (q & 0x30303030u) | (hh & 0x40404040u);
        return ((q >> 6) & 0x03030303u) | ((hh << 2) & 0x04040404u);
    }
    template <int j>
    static UQ_DEV int4 extract(const int4& q, const int4& hh) {
        return make_int4((int)v3<j>((uint32_t)q.x, (uint32_t)hh.x), (int)v3<j>((uint32_t)q.y, (uint32_t)hh.y),
                         (int)v3<j>((uint32_t)q.z, (uint32_t)hh.z), (int)v3<j>((uint32_t)q.w, (uint32_t)hh.w));
    }
    static UQ_DEV int4 shr1(const int4& h) {
        return make_int4((int)((uint32_t)h.x >> 1), (int)((uint32_t)h.y >> 1), (int)((uint32_t)h.z >> 1),
                         (int)((uint32_t)h.w >> 1));
    }
    struct W { int4 h0, h1, q0, q1; uint32_t sc0, sc1; uint16_t d; };
    // row base pointers (nu = 2 * superblocks per row)
    struct R { const uint8_t* blk; const uint8_t* sc; const uint16_t* d; };
    static UQ_DEV R row_ptr(const WArgs& w, int64_t row, int64_t nu) {
        const int64_t sb0 = row * (nu >> 1);
        return R{(const uint8_t*)w.qs + sb0 * 96, w.sc + sb0 * 16, w.d + sb0};
    }
    static UQ_DEV W load_u(const R& r, int u) {
        const int sb = u >> 1, n = u & 1;
        const uint8_t* blk = r.blk + sb * 96;
        const uint8_t* q = blk + 32 + 32 * n;
        const uint2 sc = *(const uint2*)(r.sc + sb * 16 + 8 * n);
        return W{uq_ntload16(blk), uq_ntload16(blk + 16), uq_ntload16(q), uq_ntload16(q + 16), sc.x, sc.y, r.d[sb]};
    }
    static UQ_DEV W load_w(const WArgs& w, int64_t row, int64_t nu, int u) { return load_u(row_ptr(w, row, nu), u); }
    // Group j of the unit: D = GS[j] * (sum of the 16 (value+4) x products)
    // - 4 * GS[j] * sum(x), started from that correction (the accumulator of
    // the first dot4); T = s0 * D0 + s1 * D1 = GS[j] * (s0 i0 + s1 i1) in
    // 24-bit multiplies (|D| <= 16 * 16 * 4 * 127 < 2^23). d*(s-32) is exact
    // in f32 (11-bit x 6-bit), so the block's (d*s0)*i0 + (d*s1)*i1 is
    // d*(s0*i0 + s1*i1), and (d / GS[j]) * T is that same double exactly.
    template <int j>
    static UQ_DEV double group(const int4& q0, const int4& q1, const int4& hh0, const int4& hh1, uint32_t scw,
                               const int4& xa, const int4& xb, int sa, int sb, double dd, double xsj) {
        constexpr int GS = j == 1 ? 4 : (j == 2 ? 16 : 1);
        const int4 w0 = extract<j>(q0, hh0), w1 = extract<j>(q1, hh1);
        const int d0 = dot16(w0, xa, uq_mul24(sa, -4 * GS));
        const int d1 = dot16(w1, xb, uq_mul24(sb, -4 * GS));
        const int b = 16 * (j & 1);
        const int t = uq_mul24((int)(int8_t)(scw >> b), d0) + uq_mul24((int)(int8_t)(scw >> (b + 8)), d1);
        return xsj * ((dd * (1.0 / GS)) * (double)t);
    }
    static UQ_DEV double dot(const W& wv, const X& x, int u) {
        const int n = u & 1;
        const double dd = (double)uq_half(wv.d);
        const int4 hh0 = n ? shr1(wv.h0) : wv.h0, hh1 = n ? shr1(wv.h1) : wv.h1;
        double acc = group<0>(wv.q0, wv.q1, hh0, hh1, wv.sc0, x.v[0], x.v[1], x.sx[0], x.sx[1], dd, x.s[0]);
        acc += group<1>(wv.q0, wv.q1, hh0, hh1, wv.sc0, x.v[2], x.v[3], x.sx[2], x.sx[3], dd, x.s[1]);
        acc += group<2>(wv.q0, wv.q1, hh0, hh1, wv.sc1, x.v[4], x.v[5], x.sx[4], x.sx[5], dd, x.s[2]);
        acc += group<3>(wv.q0, wv.q1, hh0, hh1, wv.sc1, x.v[6], x.v[7], x.sx[6], x.sx[7], dd, x.s[3]);
        return acc;
    }
    static UQ_DEV double term(const WArgs& w, int64_t row, int64_t nu, int u, const X& x) {
        return dot(load_w(w, row, nu, u), x, u);
    }
    // dot against an activation staged in LDS with its 16-value sums; block j's
    // 32 activations are read just before they are used (a compiler barrier
    // keeps the four blocks' reads from being hoisted together)
    static UQ_DEV double dot_lds(const W& wv, const int8_t* lx, const float* lxs, const int* ls16, int u) {
        const int n = u & 1;
        const double dd = (double)uq_half(wv.d);
        const int4* xv = (const int4*)(lx + (size_t)u * 128);
        const int4 hh0 = n ? shr1(wv.h0) : wv.h0, hh1 = n ? shr1(wv.h1) : wv.h1;
        double acc = 0.0;
#define UQ_Q3K_GROUP(J, SCW)                                                                                    \
        {                                                                                                        \
            asm volatile("" ::: "memory");                                                                       \
            const int4 xa = xv[2 * J], xb = xv[2 * J + 1];                                                       \
            const int sa = ls16[8 * u + 2 * J], sb = ls16[8 * u + 2 * J + 1];                                    \
            acc += group<J>(wv.q0, wv.q1, hh0, hh1, SCW, xa, xb, sa, sb, dd, (double)lxs[4 * u + J]);            \
        }
        UQ_Q3K_GROUP(0, wv.sc0)
        UQ_Q3K_GROUP(1, wv.sc0)
        UQ_Q3K_GROUP(2, wv.sc1)
        UQ_Q3K_GROUP(3, wv.sc1)
#undef UQ_Q3K_GROUP
        return acc;
    }
    // ggml Q3_K 6-bit scale k (0..15) of the 12 packed bytes b
    static UQ_DEV int scale6_k(const uint8_t* b, int k) {
        const int low = k < 8 ? (b[k] & 0xF) : (b[k - 8] >> 4);
        const int high = (b[8 + (k & 3)] >> (2 * (k >> 2))) & 3;
        return low | (high << 4);
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
