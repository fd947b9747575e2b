// GGUF block-quant matvec for gfx950 (Q8_0, Q4_K, Q3_K) with int8 activations.
//
// Replaces linear_dp4a / qkv_dp4a / gateup_dp4a (driver/kernels/gpu_dp4a.cu:23-64)
// and the fp32-activation frontier_matvec (driver/kernels/frontier_quant.cu:58-66).
//
// Design (bandwidth-bound, no MFMA):
//  * weights are repacked once so every lane issues 16-byte global loads:
//    Q8_0 -> int8 plane [rows][K] + fp16 scale plane; Q4_K -> 128-byte nibble
//    plane + 16 unpacked scale/min bytes + d|dmin per superblock; Q3_K -> 96-byte quant
//    plane + 16 unpacked signed scale bytes + fp16 d plane. Each repack is checked by
//    rebuilding the GGUF bytes on the device.
//  * a row is owned by LPR consecutive lanes of a wave64; lane `sub` handles
//    work units sub, sub+LPR, ... (Q8_0 unit = 16 values, Q4_K = 64, Q3_K = 128).
//    The lane's activation units are loaded into registers once and reused for
//    every row the wave visits (grid-stride over row sets).
//  * int32 per-block dots with v_dot4_i32_i8; each block contributes an exact
//    double term, lanes are combined by a butterfly in double, one f32 rounding.
#include "uq_device.h"
#include "uq_internal.h"
#include "uq_units.h"

namespace uq {
namespace {

constexpr int WG = 256;  // 4 waves

// ---------------------------------------------------------------- activation quant
__global__ __launch_bounds__(WG) void k_quant_act(const float* __restrict__ x, int64_t n,
                                                  int8_t* __restrict__ xq, float* __restrict__ xs) {
    const int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x;
    const float v = i < n ? x[i] : 0.0f;  // n % 32 == 0: a 32-lane block is all in or all out
    float s;
    const int8_t q = uq_quant_lane(v, &s);
    if (i < n) {
        xq[i] = q;
        if ((threadIdx.x & 31) == 0) xs[i >> 5] = s;
    }
}

// ---------------------------------------------------------------- repack / verify
// Q8_0: 34-byte GGUF block (fp16 d, 32 x int8) -> qs[row][32b..] + d[row][b].
__global__ __launch_bounds__(WG) void k_q8_repack(const uint8_t* __restrict__ src, int64_t rows, int64_t nb,
                                                  int8_t* __restrict__ qs, uint16_t* __restrict__ d) {
    const int64_t blk = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (blk >= rows * nb) return;
    const uint8_t* p = src + blk * 34;
    d[blk] = (uint16_t)(p[0] | (p[1] << 8));
    uint32_t w[8];
#pragma unroll
    for (int k = 0; k < 8; k++)
        w[k] = (uint32_t)p[2 + 4 * k] | ((uint32_t)p[3 + 4 * k] << 8) | ((uint32_t)p[4 + 4 * k] << 16) |
               ((uint32_t)p[5 + 4 * k] << 24);
    int4* dst = (int4*)(qs + blk * 32);
    dst[0] = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
    dst[1] = make_int4((int)w[4], (int)w[5], (int)w[6], (int)w[7]);
}
// Rebuilds each GGUF block from the planes and counts differing bytes
// (the byte-for-byte check of gpu_prefill.rs:74-93).
__global__ __launch_bounds__(WG) void k_q8_verify(const int8_t* __restrict__ qs, const uint16_t* __restrict__ d,
                                                  const uint8_t* __restrict__ src, int64_t rows, int64_t nb,
                                                  unsigned* __restrict__ bad) {
    const int64_t blk = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (blk >= rows * nb) return;
    const uint8_t* p = src + blk * 34;
    unsigned miss = 0;
    miss += (uint8_t)(d[blk] & 0xff) != p[0];
    miss += (uint8_t)(d[blk] >> 8) != p[1];
    for (int j = 0; j < 32; j++) miss += (uint8_t)qs[blk * 32 + j] != p[2 + j];
    if (miss) atomicAdd(bad, miss);
}
// Q4_K: 144-byte GGUF superblock (d, dmin, 12 packed scale/min bytes, qs 128)
// -> nibble plane, scm[blk][4 pairs][4] (scale 2j, scale 2j+1, min 2j, min
// 2j+1 as bytes) and
// dm[blk] = d | dmin. In the nibble plane byte b of unit u (32 bytes of qs,
// u = 4 * superblock-in-row + pair) of row r sits at r*nu*32 + (b/16)*nu*16 +
// u*16 + b%16 (nu units per row). The verify kernel packs everything back.
__device__ __forceinline__ int64_t q4k_qoff(int64_t blk, int64_t spr, int j, int b) {
    const int64_t row = blk / spr, nu = 4 * spr, u = 4 * (blk % spr) + j;
    return row * nu * 32 + (b >> 4) * nu * 16 + u * 16 + (b & 15);
}
__global__ __launch_bounds__(WG) void k_q4k_repack(const uint8_t* __restrict__ src, int64_t blocks, int64_t spr,
                                                   int8_t* __restrict__ q, uint8_t* __restrict__ scm,
                                                   uint32_t* __restrict__ dm) {
    const int64_t blk = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (blk >= blocks) return;
    const uint8_t* p = src + blk * 144;
    uint8_t* dq = (uint8_t*)q;
    dm[blk] = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    for (int j = 0; j < 4; j++) {
        int s0, m0, s1, m1;
        Q4K::scale_min_k4(p + 4, 2 * j, s0, m0);
        Q4K::scale_min_k4(p + 4, 2 * j + 1, s1, m1);
        uint8_t* o = scm + blk * 16 + 4 * j;
        o[0] = (uint8_t)s0;
        o[1] = (uint8_t)s1;
        o[2] = (uint8_t)m0;
        o[3] = (uint8_t)m1;
    }
    for (int i = 0; i < 128; i++) dq[q4k_qoff(blk, spr, i >> 5, i & 31)] = p[16 + i];
}
__global__ __launch_bounds__(WG) void k_q4k_verify(const int8_t* __restrict__ q, const uint8_t* __restrict__ scm,
                                                   const uint32_t* __restrict__ dm, const uint8_t* __restrict__ src,
                                                   int64_t blocks, int64_t spr, unsigned* __restrict__ bad) {
    const int64_t blk = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (blk >= blocks) return;
    const uint8_t* p = src + blk * 144;
    uint8_t sc[8], mn[8];
    for (int k = 0; k < 8; k++) {
        sc[k] = scm[blk * 16 + 4 * (k >> 1) + (k & 1)];
        mn[k] = scm[blk * 16 + 4 * (k >> 1) + 2 + (k & 1)];
    }
    unsigned miss = 0;
    for (int i = 0; i < 4; i++) miss += (uint8_t)(dm[blk] >> (8 * i)) != p[i];
    for (int k = 0; k < 8; k++) miss += (sc[k] > 63) + (mn[k] > 63);
    for (int k = 0; k < 4; k++) {
        miss += (uint8_t)(sc[k] | ((sc[k + 4] >> 4) << 6)) != p[4 + k];
        miss += (uint8_t)(mn[k] | ((mn[k + 4] >> 4) << 6)) != p[8 + k];
        miss += (uint8_t)((sc[k + 4] & 0xF) | ((mn[k + 4] & 0xF) << 4)) != p[12 + k];
    }
    for (int i = 0; i < 128; i++) miss += (uint8_t)q[q4k_qoff(blk, spr, i >> 5, i & 31)] != p[16 + i];
    if (miss) atomicAdd(bad, miss);
}
// Q3_K: 110-byte GGUF superblock (hmask 32, qs 64, 12 packed scale bytes, d 2)
// -> four 64-value units (Q3K::pack_unit): q[blk][4][16] (words A), p[blk][4][16]
// (words B, the four scales - 32, d). The verify kernel rebuilds the GGUF
// bytes from the planes (hmask, qs, the 12 scale bytes, d in every unit).
__global__ __launch_bounds__(WG) void k_q3k_repack(const uint8_t* __restrict__ src, int64_t blocks,
                                                   int8_t* __restrict__ q, int8_t* __restrict__ sc,
                                                   uint16_t* __restrict__ d) {
    const int64_t blk = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (blk >= blocks) return;
    const uint8_t* g = src + blk * 110;
    uint32_t* qa = (uint32_t*)q + blk * 16;
    uint32_t* pw = (uint32_t*)sc + blk * 16;
    for (int p = 0; p < 4; p++) {
        uint32_t A[4], P[4];
        Q3K::pack_unit(g, p, A, P);
        for (int t = 0; t < 4; t++) qa[4 * p + t] = A[t];
        for (int k = 0; k < 4; k++) pw[4 * p + k] = P[k];
    }
}
// Bytes of GGUF superblock g that the four units' words A, P do not rebuild
// (hmask, qs, the 12 scale bytes, d in every unit).
__device__ unsigned q3k_units_miss(const uint32_t (&A4)[4][4], const uint32_t (&P4)[4][4], const uint8_t* g) {
    uint8_t hm[32] = {}, qs[64] = {};
    int v[16];
    unsigned miss = 0;
    for (int p = 0; p < 4; p++) {
        const uint32_t* A = A4[p];
        const uint32_t* P = P4[p];
        miss += P[3] != ((uint32_t)g[108] | (uint32_t)g[109] << 8);
        for (int c = 0; c < 4; c++) {
            v[4 * p + c] = (int)(int8_t)(P[2] >> (8 * c)) + 32;
            for (int t = 0; t < 4; t++)
                for (int b = 0; b < 4; b++) {
                    int low2, hbit;
                    Q3K::unit_parts(A, P, c, t, b, low2, hbit);
                    const int i = 64 * p + 16 * c + 4 * t + b, n = i >> 7, j = (i >> 5) & 3, l = i & 31;
                    qs[32 * n + l] |= (uint8_t)(low2 << (2 * j));
                    hm[l] |= (uint8_t)(hbit << (4 * n + j));
                }
        }
    }
    for (int j = 0; j < 32; j++) miss += hm[j] != g[j];
    for (int j = 0; j < 64; j++) miss += qs[j] != g[32 + j];
    for (int k = 0; k < 16; k++) miss += v[k] < 0 || v[k] > 63;
    for (int k = 0; k < 8; k++) miss += (uint8_t)((v[k] & 0xF) | ((v[k + 8] & 0xF) << 4)) != g[96 + k];
    for (int m = 0; m < 4; m++) {
        int b = 0;
        for (int gr = 0; gr < 4; gr++) b |= ((v[4 * gr + m] >> 4) & 3) << (2 * gr);
        miss += (uint8_t)b != g[104 + m];
    }
    return miss;
}
__global__ __launch_bounds__(WG) void k_q3k_verify(const int8_t* __restrict__ q, const int8_t* __restrict__ sc,
                                                   const uint16_t* __restrict__ d, const uint8_t* __restrict__ src,
                                                   int64_t blocks, unsigned* __restrict__ bad) {
    const int64_t blk = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (blk >= blocks) return;
    const uint32_t* qa = (const uint32_t*)q + blk * 16;
    const uint32_t* pw = (const uint32_t*)sc + blk * 16;
    uint32_t A[4][4], P[4][4];
    for (int p = 0; p < 4; p++)
        for (int t = 0; t < 4; t++) {
            A[p][t] = qa[4 * p + t];
            P[p][t] = pw[4 * p + t];
        }
    const unsigned miss = q3k_units_miss(A, P, src + blk * 110);
    if (miss) atomicAdd(bad, miss);
}

// Row-block layout (Q3KSB): one thread per GGUF superblock writes its P
// pieces; the verify kernel rebuilds the GGUF bytes from the pieces. The
// padding slots of the allocation are zeroed before the repack.
struct SbArgs {
    int S, LB, RB;
};
__global__ __launch_bounds__(WG) void k_q3k_sb_repack(const uint8_t* __restrict__ src, int64_t blocks, SbArgs g,
                                                      uint8_t* __restrict__ dst) {
    const int64_t blk = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (blk >= blocks) return;
    const int64_t r = blk / g.S;
    const int sbi = (int)(blk - r * g.S);
    uint32_t A[4][4], P[4][4], w[28];
    for (int u = 0; u < 4; u++) Q3K::pack_unit(src + blk * 110, u, A[u], P[u]);
    Q3KSB::pack(A, P, w);
    for (int k = 0; k < Q3KSB::P; k++)
        *(int4*)(dst + sb_piece(r, sbi, k, g.S, g.LB, g.RB, Q3KSB::P)) =
            make_int4((int)w[4 * k], (int)w[4 * k + 1], (int)w[4 * k + 2], (int)w[4 * k + 3]);
}
__global__ __launch_bounds__(WG) void k_q3k_sb_verify(const uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                                      int64_t blocks, SbArgs g, unsigned* __restrict__ bad) {
    const int64_t blk = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (blk >= blocks) return;
    const int64_t r = blk / g.S;
    const int sbi = (int)(blk - r * g.S);
    uint32_t w[28], A[4][4], P[4][4];
    for (int k = 0; k < Q3KSB::P; k++) {
        const int4 v = *(const int4*)(dst + sb_piece(r, sbi, k, g.S, g.LB, g.RB, Q3KSB::P));
        w[4 * k] = (uint32_t)v.x;
        w[4 * k + 1] = (uint32_t)v.y;
        w[4 * k + 2] = (uint32_t)v.z;
        w[4 * k + 3] = (uint32_t)v.w;
    }
    Q3KSB::unpack(w, A, P);
    // the 2 bytes after d are padding and hold zero
    unsigned miss = q3k_units_miss(A, P, src + blk * 110) + ((w[27] >> 16) != 0);
    if (miss) atomicAdd(bad, miss);
}

// ---------------------------------------------------------------- matvec kernel

// One row of a lane group: every weight load of the row is issued, then the
// dots run (a unit past the row end loads the last unit and is dropped by a
// select), the lane group reduces, lane 0 stores.
template <class KQ, int LPR, int NBL, bool GATEUP>
__device__ __forceinline__ void matvec_row(const WArgs& w, const WArgs& w2, const typename KQ::X* xr, float* y,
                                           int64_t row, int64_t end, int64_t nu, int sub) {
    // rows past the end load the last row; every lane takes part in the reductions
    const int64_t rr = row < end ? row : end - 1;
    typename KQ::W wv[NBL], wv2[NBL];
    const typename KQ::R rp = KQ::row_ptr(w, rr, nu);
    typename KQ::R rp2{};
    if (GATEUP) rp2 = KQ::row_ptr(w2, rr, nu);
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + LPR * i, uc = u < nu ? u : (int)nu - 1;
        wv[i] = KQ::load_u(rp, uc);
        if (GATEUP) wv2[i] = KQ::load_u(rp2, uc);
    }
    double acc = 0.0, acc2 = 0.0;
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + LPR * i, uc = u < nu ? u : (int)nu - 1;
        const double t = KQ::dot(wv[i], xr[i], uc);
        acc += u < nu ? t : 0.0;
        if (GATEUP) {
            const double t2 = KQ::dot(wv2[i], xr[i], uc);
            acc2 += u < nu ? t2 : 0.0;
        }
    }
    acc = uq_group_sum<LPR>(acc);
    if (GATEUP) acc2 = uq_group_sum<LPR>(acc2);
    if (row < end && sub == 0) y[row] = GATEUP ? uq_silu_mul((float)acc, (float)acc2) : (float)acc;
}

template <class KQ, int LPR, int NBL, bool GATEUP>
__global__ __launch_bounds__(WG) void k_matvec(WArgs w, WArgs w2, const int8_t* __restrict__ xq,
                                               const float* __restrict__ xs, float* __restrict__ y,
                                               int64_t rows, int64_t K, int64_t share) {
    constexpr int RPW = 64 / LPR;
    constexpr int RPB = RPW * (WG / 64);
    const int64_t nu = K / KQ::UNIT;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, grp = lane / LPR;
    typename KQ::X xr[NBL];
    load_xr<KQ, LPR, NBL>(xr, xq, xs, nu, sub);
    if (rows <= (int64_t)gridDim.x * RPB) {
        // one pass: this workgroup's even share of the rows
        const RowSpan sp = even_span(rows, share);
        const int64_t row = sp.begin + wave * RPW + grp;
        if (sp.begin + wave * RPW < sp.end) matvec_row<KQ, LPR, NBL, GATEUP>(w, w2, xr, y, row, sp.end, nu, sub);
    } else {
        for (int64_t row0 = (int64_t)blockIdx.x * RPB; row0 < rows; row0 += (int64_t)gridDim.x * RPB)
            matvec_row<KQ, LPR, NBL, GATEUP>(w, w2, xr, y, row0 + wave * RPW + grp, rows, nu, sub);
    }
}

// Several weights with the same K and one shared x in one launch (the batch of
// llm.rs:226-245 and frontier_multi_matvec's job table): workgroup -> job by
// the ascending first-workgroup table, x loaded into registers once, then the
// job's rows exactly as k_matvec computes them (identical results).
constexpr int MV_MAX_JOBS = 8;
struct MvJob {
    WArgs w, w2;      // w2.qs != null: a gate/up pair writing silu(gate)*up
    float* y;
    int64_t rows, share;
    int32_t wg0, wgs;
};
struct MvJobs {
    MvJob job[MV_MAX_JOBS];
    int count;
};
template <class KQ, int LPR, int NBL>
__global__ __launch_bounds__(WG) void k_matvec_multi(MvJobs a, const int8_t* __restrict__ xq,
                                                     const float* __restrict__ xs, int64_t K) {
    constexpr int RPW = 64 / LPR;
    constexpr int RPB = RPW * (WG / 64);
    int lo = 0, hi = a.count;
    while (lo + 1 < hi) {
        const int mid = (lo + hi) >> 1;
        if (a.job[mid].wg0 <= (int)blockIdx.x) lo = mid;
        else hi = mid;
    }
    const MvJob& j = a.job[lo];
    const int wgi = (int)blockIdx.x - j.wg0;
    const int64_t nu = K / KQ::UNIT;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, grp = lane / LPR;
    typename KQ::X xr[NBL];
    load_xr<KQ, LPR, NBL>(xr, xq, xs, nu, sub);
    const bool pair = j.w2.qs != nullptr;
    if (j.rows <= (int64_t)j.wgs * RPB) {
        // one pass: this workgroup's even share of the job's rows
        const RowSpan sp = even_span_of(j.rows, j.share, wgi, j.wgs);
        const int64_t row = sp.begin + wave * RPW + grp;
        if (sp.begin + wave * RPW < sp.end) {
            if (pair) matvec_row<KQ, LPR, NBL, true>(j.w, j.w2, xr, j.y, row, sp.end, nu, sub);
            else matvec_row<KQ, LPR, NBL, false>(j.w, j.w2, xr, j.y, row, sp.end, nu, sub);
        }
    } else {
        for (int64_t row0 = (int64_t)wgi * RPB; row0 < j.rows; row0 += (int64_t)j.wgs * RPB) {
            if (pair) matvec_row<KQ, LPR, NBL, true>(j.w, j.w2, xr, j.y, row0 + wave * RPW + grp, j.rows, nu, sub);
            else matvec_row<KQ, LPR, NBL, false>(j.w, j.w2, xr, j.y, row0 + wave * RPW + grp, j.rows, nu, sub);
        }
    }
}

// One row with the activation read from LDS (K-quant units), same order of
// work as matvec_row.
template <class KQ, int LPR, int NBL, bool GATEUP>
__device__ __forceinline__ void matvec_row_lds(const WArgs& w, const WArgs& w2, const int8_t* lx, const float* lxs,
                                               const int* ls16, float* y, int64_t row, int64_t end, int64_t nu,
                                               int sub) {
    const int64_t rr = row < end ? row : end - 1;
    typename KQ::W wv[NBL], wv2[NBL];
    const typename KQ::R rp = KQ::row_ptr(w, rr, nu);
    typename KQ::R rp2{};
    if (GATEUP) rp2 = KQ::row_ptr(w2, rr, nu);
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + LPR * i, uc = u < nu ? u : (int)nu - 1;
        wv[i] = KQ::load_u(rp, uc);
        if (GATEUP) wv2[i] = KQ::load_u(rp2, uc);
    }
    double acc = 0.0, acc2 = 0.0;
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + LPR * i, uc = u < nu ? u : (int)nu - 1;
        asm volatile("" ::: "memory");  // one unit's activation reads at a time
        const double t = KQ::dot_lds(wv[i], lx, lxs, ls16, uc);
        acc += u < nu ? t : 0.0;
        if (GATEUP) {
            const double t2 = KQ::dot_lds(wv2[i], lx, lxs, ls16, uc);
            acc2 += u < nu ? t2 : 0.0;
        }
    }
    acc = uq_group_sum<LPR>(acc);
    if (GATEUP) acc2 = uq_group_sum<LPR>(acc2);
    if (row < end && sub == 0) y[row] = GATEUP ? uq_silu_mul((float)acc, (float)acc2) : (float)acc;
}

// K-quant variant: units carry 64-128 activation values, too many to keep in
// registers across rows, so the workgroup stages the quantized activation,
// its scales and its 16-value sums in LDS once and each unit reads its slice
// from LDS right before its dot. K <= MAX_XL.
constexpr int MAX_XL = 16384;
template <class KQ, int LPR, int NBL, bool GATEUP>
__global__ __launch_bounds__(WG) void k_matvec_xl(WArgs w, WArgs w2, const int8_t* __restrict__ xq,
                                                  const float* __restrict__ xs, float* __restrict__ y,
                                                  int64_t rows, int64_t K, int64_t share) {
    // dynamic LDS sized to K (xl_lds_bytes): x (K int8), its scales (K/32 f32), its 16-value sums (K/16
    // int, as KQ::stage16 forms them)
    extern __shared__ __attribute__((aligned(16))) int8_t xl_lds[];
    int8_t* lx = xl_lds;
    float* lxs = (float*)(xl_lds + K);
    int* ls16 = (int*)(xl_lds + K + K / 8);
    constexpr int RPW = 64 / LPR;
    constexpr int RPB = RPW * (WG / 64);
    const int64_t nu = K / KQ::UNIT;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, grp = lane / LPR;
    for (int g = threadIdx.x; g < K / 16; g += WG) {
        const int4 v = ((const int4*)xq)[g];
        ((int4*)lx)[g] = v;
        const int ones = 0x01010101;
        int c = uq_dot4(ones, v.x, 0);
        c = uq_dot4(ones, v.y, c);
        c = uq_dot4(ones, v.z, c);
        ls16[g] = KQ::stage16(g, uq_dot4(ones, v.w, c));
    }
    for (int b = threadIdx.x; b < K / 32; b += WG) lxs[b] = xs[b];
    __syncthreads();
    if (rows <= (int64_t)gridDim.x * RPB) {
        // one pass: this workgroup's even share of the rows
        const RowSpan sp = even_span(rows, share);
        if (sp.begin + wave * RPW < sp.end)
            matvec_row_lds<KQ, LPR, NBL, GATEUP>(w, w2, lx, lxs, ls16, y, sp.begin + wave * RPW + grp, sp.end, nu, sub);
    } else {
        for (int64_t row0 = (int64_t)blockIdx.x * RPB; row0 < rows; row0 += (int64_t)gridDim.x * RPB)
            matvec_row_lds<KQ, LPR, NBL, GATEUP>(w, w2, lx, lxs, ls16, y, row0 + wave * RPW + grp, rows, nu, sub);
    }
}

// ---------------------------------------------------------------- row-block matvec
// Q3KSB layout: lane t owns slot t % LB of row block
// blockIdx.x * (blockDim.x / LB) + t / LB, i.e. one superblock of one row, and
// loads its P pieces, each wave instruction covering 1 KB of consecutive
// bytes. The activation, its scales and its 16-value sums are staged in LDS
// per superblock with strides of 272, 48 and 80 bytes, so the 16-byte reads
// of lanes on different superblocks fall on different banks. Each lane's
// double term goes to LDS and one thread per row adds its row's S terms in
// superblock order (the same exact double terms as the unit kernels; only
// the order of the double additions differs).
constexpr int SB_X = 272, SB_XS = 12, SB_S16 = 20;
inline size_t sb_lds_bytes(int S, int nthr, bool pair) {
    return (size_t)S * (SB_X + 4 * SB_XS + 4 * SB_S16) + (size_t)nthr * 8 * (pair ? 2 : 1);
}
template <class KS> struct SbDot;
template <> struct SbDot<Q3KSB> {
    static UQ_DEV int stage16(int g, int sum) { return Q3K::gs_corr(g & 3, sum); }
    static UQ_DEV double dot(const int4 (&w)[Q3KSB::P], const int8_t* lx, const float* lxs, const int* l16) {
        const double dd = (double)uq_half((uint16_t)((uint32_t)w[6].w & 0xffff));
        double acc = 0.0;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int4 A = w[u], Bq = w[4 + (u >> 1)];
            const uint32_t B0 = (uint32_t)((u & 1) ? Bq.z : Bq.x), B1 = (uint32_t)((u & 1) ? Bq.w : Bq.y);
            const int4* xp = (const int4*)(lx + 64 * u);
            const int4 xv[4] = {xp[0], xp[1], xp[2], xp[3]};
            const int4 c = *(const int4*)(l16 + 4 * u);
            const float2 xs = *(const float2*)(lxs + 2 * u);
            int D0 = c.x, D1 = c.y, D2 = c.z, D3 = c.w;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                int wd[4];
                Q3K::words((uint32_t)Q3K::lane4(A, t), t < 2 ? B0 : B1, t, wd);
                D0 = uq_dot4(wd[0], Q3K::lane4(xv[0], t), D0);
                D1 = uq_dot4(wd[1], Q3K::lane4(xv[1], t), D1);
                D2 = uq_dot4(wd[2], Q3K::lane4(xv[2], t), D2);
                D3 = uq_dot4(wd[3], Q3K::lane4(xv[3], t), D3);
            }
            const uint32_t win = Q3KSB::scale_window((uint32_t)w[6].x, (uint32_t)w[6].y, (uint32_t)w[6].z, u);
            const int s0 = Q3KSB::scale_field(win, 0), s1 = Q3KSB::scale_field(win, 1);
            const int s2 = Q3KSB::scale_field(win, 2), s3 = Q3KSB::scale_field(win, 3);
            const int T0 = uq_mul24(s0, D0) + uq_mul24(s1, D1);
            const int T1 = uq_mul24(s2, D2) + uq_mul24(s3, D3);
            acc += (dd * (double)xs.x) * (double)T0 + (dd * ((double)xs.y * (1.0 / 16))) * (double)T1;
        }
        return acc;
    }
};

template <class KS, bool GATEUP>
__global__ __launch_bounds__(WG) void k_matvec_sb(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2,
                                                  const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                  float* __restrict__ y, int64_t rows, int64_t blocks, SbArgs g) {
    extern __shared__ __attribute__((aligned(16))) int8_t sb_lds[];
    constexpr int P = KS::P;
    const int S = g.S, LB = g.LB, RB = g.RB, K = 256 * S;
    int8_t* lx = sb_lds;
    float* lxs = (float*)(sb_lds + S * SB_X);
    int* l16 = (int*)(lxs + SB_XS * S);
    double* part = (double*)(l16 + SB_S16 * S);
    const int tid = threadIdx.x, nthr = blockDim.x, bpw = nthr / LB;
    for (int gi = tid; gi < K / 16; gi += nthr) {
        const int4 v = ((const int4*)xq)[gi];
        const int sb = gi >> 4, wi = gi & 15;
        *(int4*)(lx + sb * SB_X + 16 * wi) = v;
        l16[sb * SB_S16 + wi] = SbDot<KS>::stage16(wi, Q3K::sum16(v));
    }
    for (int b = tid; b < K / 32; b += nthr) lxs[(b >> 3) * SB_XS + (b & 7)] = xs[b];
    __syncthreads();
    const int64_t blk = (int64_t)blockIdx.x * bpw + tid / LB;
    const int j = tid % LB, rr = j / S, s = j - rr * S;
    const bool valid = rr < RB && blk * RB + rr < rows;
    // a block past the last one (grid rounding) reads the last block's slot
    const int64_t bl = blk < blocks ? blk : blocks - 1;
    const uint8_t* base = w + (bl * P * LB + j) * 16;
    int4 wv[P], wv2[P];
#pragma unroll
    for (int k = 0; k < P; k++) wv[k] = uq_ntload16(base + (int64_t)k * LB * 16);
    if (GATEUP) {
        const uint8_t* base2 = w2 + (bl * P * LB + j) * 16;
#pragma unroll
        for (int k = 0; k < P; k++) wv2[k] = uq_ntload16(base2 + (int64_t)k * LB * 16);
    }
    const int8_t* xsb = lx + s * SB_X;
    const float* xssb = lxs + s * SB_XS;
    const int* s16 = l16 + s * SB_S16;
    const double v = SbDot<KS>::dot(wv, xsb, xssb, s16);
    part[tid] = valid ? v : 0.0;
    if (GATEUP) {
        const double v2 = SbDot<KS>::dot(wv2, xsb, xssb, s16);
        part[nthr + tid] = valid ? v2 : 0.0;
    }
    __syncthreads();
    if (tid < bpw * RB) {
        const int bb = tid / RB, r = tid - bb * RB;
        const int64_t row = ((int64_t)blockIdx.x * bpw + bb) * RB + r;
        if (row < rows) {
            const double* pr = part + bb * LB + r * S;
            double a = 0.0, a2 = 0.0;
            for (int q = 0; q < S; q++) a += pr[q];
            if (GATEUP) {
                for (int q = 0; q < S; q++) a2 += pr[nthr + q];
                y[row] = uq_silu_mul((float)a, (float)a2);
            } else {
                y[row] = (float)a;
            }
        }
    }
}

// Integer per-block dots (test surface for the int32 work): Q8_0 per 32-block,
// Q4_K per 32 sub-block (q 0..15), Q3_K per 16 sub-block (q3 -4..3); one thread
// per (row, block), using the same int8 dot primitive as the matvec.
__global__ __launch_bounds__(WG) void k_block_dots(WArgs w, uint32_t kind, const int8_t* __restrict__ xq,
                                                   int32_t* __restrict__ dots, int64_t rows, int64_t K, SbArgs sb) {
    const int bsz = kind == KIND_Q3_K ? 16 : 32;
    const int64_t nb = K / bsz;
    const int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (i >= rows * nb) return;
    const int64_t row = i / nb, b = i % nb;
    const int8_t* x = xq + b * bsz;
    int c = 0;
    if (sb.LB) {
        // row-block layout (Q3_K): the superblock's pieces, then its unit words
        const int sbi = (int)(b / 16), k = (int)(b % 16);
        uint32_t wd[4 * Q3KSB::P];
        for (int p = 0; p < Q3KSB::P; p++) {
            const int4 v = *(const int4*)((const uint8_t*)w.qs + sb_piece(row, sbi, p, sb.S, sb.LB, sb.RB, Q3KSB::P));
            wd[4 * p] = (uint32_t)v.x;
            wd[4 * p + 1] = (uint32_t)v.y;
            wd[4 * p + 2] = (uint32_t)v.z;
            wd[4 * p + 3] = (uint32_t)v.w;
        }
        const int* xp = (const int*)x;
        uint32_t A[4][4], Pw[4][4];
        Q3KSB::unpack(wd, A, Pw);
        const int u = k >> 2, cc = k & 3;
        for (int t = 0; t < 4; t++) {
            int v = 0;
            for (int bb = 0; bb < 4; bb++) {
                int low2, hbit;
                Q3K::unit_parts(A[u], Pw[u], cc, t, bb, low2, hbit);
                v |= (low2 | hbit << 2) << (8 * bb);
            }
            c = uq_dot4(v, xp[t], c);
            c -= 4 * uq_dot4(0x01010101, xp[t], 0);
        }
        dots[i] = c;
        return;
    }
    if (kind == KIND_Q8_0) {
        const int4* p = (const int4*)(w.qs + i * 32);
        const int4* xp = (const int4*)x;
        c = uq_dot32(p[0], p[1], xp[0], xp[1]);
    } else if (kind == KIND_Q4_K) {
        const int64_t nu = K / 64, u = (b / 8) * 4 + ((b % 8) >> 1);
        const int h = (int)(b & 1);
        const uint8_t* qs = (const uint8_t*)w.qs + row * nu * 32 + u * 16;
        const int* xp = (const int*)x;
        for (int k = 0; k < 8; k++) {
            const int wq = *(const int*)(qs + (k >> 2) * nu * 16 + 4 * (k & 3));
            c = uq_dot4(h ? Q4K::hi4(wq) : Q4K::lo4(wq), xp[k], c);
        }
    } else {
        // sub-block b of the row: unit (superblock b / 16, p = (b / 4) % 4), sub-block c = b % 4 of the unit
        const int64_t un = (row * (K / 256)) * 4 + b / 4;
        const int cc = (int)(b & 3);
        const uint32_t* qa = (const uint32_t*)w.qs + un * 4;
        const uint32_t* pw = (const uint32_t*)w.sc + un * 4;
        const uint32_t A[4] = {qa[0], qa[1], qa[2], qa[3]};
        const uint32_t P[4] = {pw[0], pw[1], pw[2], pw[3]};
        const int* xp = (const int*)x;
        for (int t = 0; t < 4; t++) {
            int v = 0;
            for (int bb = 0; bb < 4; bb++) {
                int low2, hbit;
                Q3K::unit_parts(A, P, cc, t, bb, low2, hbit);
                v |= (low2 | hbit << 2) << (8 * bb);
            }
            c = uq_dot4(v, xp[t], c);
            c -= 4 * uq_dot4(0x01010101, xp[t], 0);
        }
    }
    dots[i] = c;
}

inline unsigned grid_for(int64_t items, int per_block) {
    return (unsigned)((items + per_block - 1) / per_block);
}

inline size_t xl_lds_bytes(int64_t K) { return (size_t)K + (size_t)K / 8 + (size_t)K / 4; }

// Workgroups of `kern` (WG threads, `lds` dynamic LDS bytes) resident per CU,
// from the runtime's occupancy query, cached per kernel and LDS size.
int resident_blocks(const void* kern, size_t lds) {
    struct Entry { const void* k; size_t lds; int n; };
    static Entry cache[64];
    static int used = 0;
    for (int i = 0; i < used; i++)
        if (cache[i].k == kern && cache[i].lds == lds) return cache[i].n;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, WG, lds) != hipSuccess || n <= 0) n = 1;
    if (n > 8) n = 8;
    if (used < 64) cache[used++] = Entry{kern, lds, n};
    return n;
}

template <class KQ, int LPR, int NBL, bool XL = false>
void launch_t(const Weight& w, const Weight* w2, const int8_t* xq, const float* xs, float* y, hipStream_t s) {
    constexpr int RPB = (64 / LPR) * (WG / 64);
    const size_t lds = XL ? xl_lds_bytes(w.n) : 0;
    const void* kern;
    if constexpr (XL) kern = w2 ? (const void*)k_matvec_xl<KQ, LPR, NBL, true> : (const void*)k_matvec_xl<KQ, LPR, NBL, false>;
    else kern = w2 ? (const void*)k_matvec<KQ, LPR, NBL, true> : (const void*)k_matvec<KQ, LPR, NBL, false>;
    // a multiple of the CU count with at most one pass of rows per workgroup
    // while that fits on the chip at once. Past that (lm_head), Q8_0 and Q4_K
    // take one row block per workgroup and leave the balancing to the
    // dispatcher, which refills a CU as its workgroups retire: measured faster
    // than resident workgroups striding over the rows (Q8_0 lm_head 81% -> 85%
    // of HBM peak).
    const int64_t cu = cu_count(), m = (w.m + cu * RPB - 1) / (cu * RPB);
    const int64_t fit = cu * resident_blocks(kern, lds);
    const int64_t nblk = (w.m + RPB - 1) / RPB;
    int64_t g = m * cu;
    if (g > fit) g = nblk;
    if (g > w.m) g = w.m;
    const unsigned grid = (unsigned)g;
    const int64_t share = w.m / g;
    WArgs a{w.qs, w.d, w.sc}, b{nullptr, nullptr, nullptr};
    if (w2) b = WArgs{w2->qs, w2->d, w2->sc};
    if constexpr (XL) {
        if (w2) hipLaunchKernelGGL((k_matvec_xl<KQ, LPR, NBL, true>), dim3(grid), dim3(WG), lds, s, a, b, xq, xs, y, w.m, w.n, share);
        else hipLaunchKernelGGL((k_matvec_xl<KQ, LPR, NBL, false>), dim3(grid), dim3(WG), lds, s, a, b, xq, xs, y, w.m, w.n, share);
    } else {
        if (w2) hipLaunchKernelGGL((k_matvec<KQ, LPR, NBL, true>), dim3(grid), dim3(WG), 0, s, a, b, xq, xs, y, w.m, w.n, share);
        else hipLaunchKernelGGL((k_matvec<KQ, LPR, NBL, false>), dim3(grid), dim3(WG), 0, s, a, b, xq, xs, y, w.m, w.n, share);
    }
}

// Row-block layout: one block per LB-lane group, the largest group count per
// workgroup (of 256 threads at most) that still gives two workgroups per CU.
template <class KS>
int launch_sb(const Weight& w, const Weight* w2, const int8_t* xq, const float* xs, float* y, hipStream_t s) {
    const SbGeom g = sb_geom(w.n, w.m);
    if (g.LB != w.sb_lb || g.RB != w.sb_rb || (w2 && (w2->sb_lb != w.sb_lb || w2->sb_rb != w.sb_rb)))
        return set_error(ERR_SHAPE, "matvec: row-block geometry differs from the upload's");
    int bpw = WG / g.LB;
    while (bpw > 1 && (g.blocks + bpw - 1) / bpw < 2 * (int64_t)cu_count()) bpw /= 2;
    const int nthr = bpw * g.LB;
    const unsigned grid = (unsigned)((g.blocks + bpw - 1) / bpw);
    const size_t lds = sb_lds_bytes(g.S, nthr, w2 != nullptr);
    const SbArgs a{g.S, g.LB, g.RB};
    const uint8_t* q = (const uint8_t*)w.qs;
    if (w2)
        hipLaunchKernelGGL((k_matvec_sb<KS, true>), dim3(grid), dim3(nthr), lds, s, q, (const uint8_t*)w2->qs, xq, xs, y,
                           w.m, g.blocks, a);
    else
        hipLaunchKernelGGL((k_matvec_sb<KS, false>), dim3(grid), dim3(nthr), lds, s, q, nullptr, xq, xs, y, w.m,
                           g.blocks, a);
    return OK;
}

// Lane-group size per row from the number of units per row: small rows use
// short groups (more rows per wave), long rows spread over a full wave.
template <class KQ>
int launch_kind(const Weight& w, const Weight* w2, const int8_t* xq, const float* xs, float* y, hipStream_t s) {
    const int64_t nu = w.n / KQ::UNIT;
#define UQ_TRY(L, B) \
    if (nu <= (int64_t)(L) * (B)) { launch_t<KQ, L, B>(w, w2, xq, xs, y, s); return OK; }
    // K-quants: activation staged in LDS, lane groups sized to fit the row
#define UQ_TRYX(L, B) \
    if (nu <= (int64_t)(L) * (B)) { launch_t<KQ, L, B, true>(w, w2, xq, xs, y, s); return OK; }
    if constexpr (KQ::UNIT >= 64) {
        if (w.n <= MAX_XL) {
            UQ_TRYX(4, 1) UQ_TRYX(4, 2) UQ_TRYX(4, 3) UQ_TRYX(8, 3) UQ_TRYX(8, 4) UQ_TRYX(16, 3) UQ_TRYX(32, 3) UQ_TRYX(64, 3)
            UQ_TRYX(64, 4) UQ_TRYX(64, 6) UQ_TRYX(64, 8)
        }
    }
#undef UQ_TRYX
    UQ_TRY(4, 1) UQ_TRY(4, 2)
    UQ_TRY(8, 1) UQ_TRY(8, 2) UQ_TRY(8, 3)
    UQ_TRY(16, 2) UQ_TRY(16, 3) UQ_TRY(16, 4)
    UQ_TRY(32, 3) UQ_TRY(32, 4)
    UQ_TRY(64, 3) UQ_TRY(64, 4) UQ_TRY(64, 5) UQ_TRY(64, 6) UQ_TRY(64, 7) UQ_TRY(64, 8)
    UQ_TRY(64, 9) UQ_TRY(64, 10) UQ_TRY(64, 12) UQ_TRY(64, 14) UQ_TRY(64, 16)
#undef UQ_TRY
    return set_error(ERR_SHAPE, "matvec: input length too large");
}

}  // namespace

int cu_count() {
    static int n = 0;
    if (!n) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            return 256;
        n = v;
    }
    return n;
}

void launch_quant_act(const float* x, int64_t n, int8_t* xq, float* xs, hipStream_t s) {
    hipLaunchKernelGGL(k_quant_act, dim3(grid_for(n, WG)), dim3(WG), 0, s, x, n, xq, xs);
}
void launch_q8_repack(const uint8_t* gguf, int64_t rows, int64_t nb, int8_t* qs, uint16_t* d, hipStream_t s) {
    hipLaunchKernelGGL(k_q8_repack, dim3(grid_for(rows * nb, WG)), dim3(WG), 0, s, gguf, rows, nb, qs, d);
}
void launch_q8_verify(const int8_t* qs, const uint16_t* d, const uint8_t* gguf, int64_t rows, int64_t nb,
                      unsigned* bad, hipStream_t s) {
    hipLaunchKernelGGL(k_q8_verify, dim3(grid_for(rows * nb, WG)), dim3(WG), 0, s, qs, d, gguf, rows, nb, bad);
}
void launch_q4k_repack(const uint8_t* gguf, int64_t blocks, int64_t spr, int8_t* q, uint8_t* scm, uint32_t* dm,
                       hipStream_t s) {
    hipLaunchKernelGGL(k_q4k_repack, dim3(grid_for(blocks, WG)), dim3(WG), 0, s, gguf, blocks, spr, q, scm, dm);
}
void launch_q4k_verify(const int8_t* q, const uint8_t* scm, const uint32_t* dm, const uint8_t* gguf, int64_t blocks,
                       int64_t spr, unsigned* bad, hipStream_t s) {
    hipLaunchKernelGGL(k_q4k_verify, dim3(grid_for(blocks, WG)), dim3(WG), 0, s, q, scm, dm, gguf, blocks, spr, bad);
}
void launch_q3k_repack(const uint8_t* gguf, int64_t blocks, int8_t* q, int8_t* sc, uint16_t* d, hipStream_t s) {
    hipLaunchKernelGGL(k_q3k_repack, dim3(grid_for(blocks, WG)), dim3(WG), 0, s, gguf, blocks, q, sc, d);
}
void launch_q3k_verify(const int8_t* q, const int8_t* sc, const uint16_t* d, const uint8_t* gguf, int64_t blocks,
                       unsigned* bad, hipStream_t s) {
    hipLaunchKernelGGL(k_q3k_verify, dim3(grid_for(blocks, WG)), dim3(WG), 0, s, q, sc, d, gguf, blocks, bad);
}
void launch_sb_repack(uint32_t kind, const uint8_t* gguf, int64_t n, int64_t m, int lb, int rb, uint8_t* dst,
                      unsigned* bad, hipStream_t s) {
    const int64_t blocks = n / 256 * m;
    const SbArgs g{(int)(n / 256), lb, rb};
    if (kind != KIND_Q3_K) return;
    hipLaunchKernelGGL(k_q3k_sb_repack, dim3(grid_for(blocks, WG)), dim3(WG), 0, s, gguf, blocks, g, dst);
    hipLaunchKernelGGL(k_q3k_sb_verify, dim3(grid_for(blocks, WG)), dim3(WG), 0, s, (const uint8_t*)dst, gguf,
                       blocks, g, bad);
}

namespace {
// The job table of weights sharing K: the resident workgroups of the chip are
// split over the jobs in proportion to their rows (at least one each, at most
// one row block per workgroup when the rows allow); a table whose rows exceed
// one resident pass gives every job one row block per workgroup.
template <class KQ, int LPR, int NBL>
void launch_multi_t(const Weight* const* ws, const Weight* const* w2s, float* const* ys, int count,
                    const int8_t* xq, const float* xs, hipStream_t s) {
    constexpr int RPB = (64 / LPR) * (WG / 64);
    const void* kern = (const void*)k_matvec_multi<KQ, LPR, NBL>;
    const int64_t fit = (int64_t)cu_count() * resident_blocks(kern, 0);
    int64_t total = 0;
    for (int i = 0; i < count; i++) total += ws[i]->m;
    MvJobs a{};
    a.count = count;
    int64_t wg = 0;
    for (int i = 0; i < count; i++) {
        const Weight& w = *ws[i];
        const int64_t need = (w.m + RPB - 1) / RPB;
        int64_t g = (fit * w.m + total / 2) / total;
        if (g < 1) g = 1;
        if (g > need || total > fit * RPB) g = need;  // past one resident pass: a row block per workgroup
        MvJob& j = a.job[i];
        j.w = WArgs{w.qs, w.d, w.sc};
        j.w2 = w2s && w2s[i] ? WArgs{w2s[i]->qs, w2s[i]->d, w2s[i]->sc} : WArgs{nullptr, nullptr, nullptr};
        j.y = ys[i];
        j.rows = w.m;
        j.wgs = (int32_t)g;
        j.share = w.m / g;
        j.wg0 = (int32_t)wg;
        wg += g;
    }
    hipLaunchKernelGGL((k_matvec_multi<KQ, LPR, NBL>), dim3((unsigned)wg), dim3(WG), 0, s, a, xq, xs, ws[0]->n);
}
}  // namespace

int launch_matvec_multi(const Weight* const* ws, const Weight* const* w2s, float* const* ys, int count,
                        const int8_t* xq, const float* xs, hipStream_t s) {
    if (count < 1 || count > MV_MAX_JOBS) return set_error(ERR_ARG, "matvec job table: 1..8 weights");
    for (int i = 0; i < count; i++) {
        if (ws[i]->kind != KIND_Q8_0 || ws[i]->n != ws[0]->n)
            return set_error(ERR_SHAPE, "matvec job table: Q8_0 weights of one input length");
        if (w2s && w2s[i] && (w2s[i]->kind != ws[i]->kind || w2s[i]->n != ws[i]->n || w2s[i]->m != ws[i]->m))
            return set_error(ERR_SHAPE, "gate/up pair: shapes differ");
    }
    // the same lane geometry as launch_kind<Q8> picks for one weight of this K
    const int64_t nu = ws[0]->n / Q8::UNIT;
#define UQ_TRYM(L, B) \
    if (nu <= (int64_t)(L) * (B)) { launch_multi_t<Q8, L, B>(ws, w2s, ys, count, xq, xs, s); return OK; }
    UQ_TRYM(4, 1) UQ_TRYM(4, 2)
    UQ_TRYM(8, 1) UQ_TRYM(8, 2) UQ_TRYM(8, 3)
    UQ_TRYM(16, 2) UQ_TRYM(16, 3) UQ_TRYM(16, 4)
    UQ_TRYM(32, 3) UQ_TRYM(32, 4)
    UQ_TRYM(64, 3) UQ_TRYM(64, 4) UQ_TRYM(64, 5) UQ_TRYM(64, 6) UQ_TRYM(64, 7) UQ_TRYM(64, 8)
    UQ_TRYM(64, 9) UQ_TRYM(64, 10) UQ_TRYM(64, 12) UQ_TRYM(64, 14) UQ_TRYM(64, 16)
#undef UQ_TRYM
    return set_error(ERR_SHAPE, "matvec: input length too large");
}

int launch_matvec(const Weight& w, const Weight* w2, const int8_t* xq, const float* xs, float* y, hipStream_t s) {
    if (w2 && (w2->kind != w.kind || w2->n != w.n || w2->m != w.m))
        return set_error(ERR_SHAPE, "gate/up pair: shapes differ");
    if (w2 && (w2->sb_lb != 0) != (w.sb_lb != 0)) return set_error(ERR_SHAPE, "gate/up pair: device layouts differ");
    switch (w.kind) {
    case KIND_Q8_0: return launch_kind<Q8>(w, w2, xq, xs, y, s);
    case KIND_Q4_K: return launch_kind<Q4K>(w, w2, xq, xs, y, s);
    case KIND_Q3_K: return w.sb_lb ? launch_sb<Q3KSB>(w, w2, xq, xs, y, s) : launch_kind<Q3K>(w, w2, xq, xs, y, s);
    default: return set_error(ERR_QUANT_TYPE, "matvec: unsupported kind");
    }
}

int launch_block_dots(const Weight& w, const int8_t* xq, int32_t* dots, hipStream_t s) {
    if (w.kind != KIND_Q8_0 && w.kind != KIND_Q4_K && w.kind != KIND_Q3_K)
        return set_error(ERR_QUANT_TYPE, "block_dots: Q8_0, Q4_K or Q3_K only");
    const int bsz = w.kind == KIND_Q3_K ? 16 : 32;
    const int64_t items = w.m * (w.n / bsz);
    WArgs a{w.qs, w.d, w.sc};
    const SbArgs sb{(int)(w.n / 256), w.sb_lb, w.sb_rb};
    hipLaunchKernelGGL(k_block_dots, dim3(grid_for(items, WG)), dim3(WG), 0, s, a, w.kind, xq, dots, w.m, w.n, sb);
    return OK;
}

}  // namespace uq
