// Q8_0 prompt prefill for gfx950: int8 MFMA GEMM with the per-32-block
// rescale, and the batched norm / quant / RoPE / causal attention around it.
//
// Replaces prefill_gemm / prefill_repack / prefill_quant / prefill_resnorm /
// prefill_rope / prefill_attention / silu_mul (driver/kernels/gpu_prefill.cu:
// 10-101, gpu_ops.cu:40-42) and the stream built by prepare_prefill
// (driver/src/gpu_prefill.rs:122-150).
//
// GEMM: y[t][r] = sum over 32-blocks b, in order, of
//   f = fmaf((float)c_b, dw[r][b] * dx[t][b], f),   c_b = sum_k qw[r][k] qx[t][k]
// (gpu_prefill.cu:29-30). c_b is one v_mfma_i32_16x16x32_i8 per block with a
// zero accumulator; the scale product dw*dx comes exact from an f32
// outer-product MFMA and the convert and fmaf run on the VALU in the
// reference's order, so results match the oracle bit for bit.
// Operands come from the row-major planes used by decode (no second weight
// copy), staged through LDS; the fp16 weight scales get a [block][row]
// transpose widened to f32, so a stage's scales are contiguous float4 loads.
#include "uq_device.h"
#include "uq_blockops.h"
#include "uq_prefill.h"
#include "uq_internal.h"

namespace uq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ scale transpose
// fp16 d[row][block] -> f32 dt[block][row] (exact widening).
__global__ __launch_bounds__(256) void k_transpose_scales(const uint16_t* __restrict__ d, int64_t rows, int64_t nb,
                                                          float* __restrict__ dt) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * nb) return;
    const int64_t r = i / nb, b = i % nb;
    dt[b * rows + r] = uq_half(d[i]);
}

// ------------------------------------------------------------------ per-token norm + quant
// One workgroup per token: x = embed(token) or x + residual (stored back),
// RMSNorm, block-32 quant into xq[t][dim] and xsT[b][t].
constexpr int PF_MAXD = 4096;  // model dim bound (uq_model_create: dim <= 4096, dim % 256 == 0)
// NC = dim / 256 chunks of 256 values, one per wave (float4 per lane, partial
// sums of squares meeting in LDS): each wave issues only its chunk's loads
// (instantiated per chunk count; a launch for the 4096 bound gave a 1536-wide
// row 12 loads per wave, half of them clamped repeats).
template <int NC>
__global__ __launch_bounds__(64 * NC) void k_pf_norm(PfNormArgs a) {
    __shared__ double part[NC];
    const int t = blockIdx.x;
    NormQuantArgs nq = a.nq;
    nq.x = a.x + (size_t)t * a.nq.dim;
    nq.residual = a.residual ? a.residual + (size_t)t * a.nq.dim : nullptr;
    nq.x_out = a.x + (size_t)t * a.nq.dim;
    if (a.tokens) nq.token = a.tokens + t;
    NormQuantSplit<NC, NC> nw;
    nw.issue(nq);
    nw.finish(nq, true, part, a.xq + (size_t)t * a.nq.dim, a.xst + t, a.mp);
}

// Block-32 quant of rows of k floats: grid (k/256, tokens).
__global__ __launch_bounds__(256) void k_pf_quant(const float* __restrict__ x, int64_t k, int mp,
                                                  int8_t* __restrict__ xq, float* __restrict__ xst) {
    const int t = blockIdx.y;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const float v = i < k ? x[(size_t)t * k + i] : 0.0f;
    float s;
    const int8_t q = uq_quant_lane(v, &s);
    if (i < k) {
        xq[(size_t)t * k + i] = q;
        if ((threadIdx.x & 31) == 0) xst[(i >> 5) * mp + t] = s;
    }
}

// ------------------------------------------------------------------ GEMM
// Workgroup tile 32 rows x 64 tokens, 4 waves of 32 rows x 16 tokens (2 MFMA
// tiles, 4 with the gate/up pair). K runs in stages of four 32-blocks (128
// values) through a ring of GR stages in LDS, filled by direct global->LDS
// loads (global_load_lds_dwordx4: lane l's 16 bytes land at base + 16 l), so
// GR-1 stages are in flight while one is computed, with no register staging.
// LDS rows are 128 bytes; 16-byte chunk c of row r sits in slot c ^ swz(r),
// which makes the 16 lanes of an MFMA fragment read hit 16 distinct bank pairs.
// MFMA 16x16x32 i8 lane layout: A lane l = row l%16, k (l/16)*8..+7; B lane l =
// token l%16, same k; D lane l = rows (l/16)*4..+3, token l%16.
// Per output and block the VALU does (float)c and the fmaf in the
// reference's order, with the scale product dw*dx from an outer-product
// MFMA; that VALU work, not the int8 MFMA, bounds this kernel.
constexpr int GK_BLK = 4;                  // 32-blocks per stage
constexpr int GBM = 32;                    // rows per workgroup tile
// Ring depth (in k_pf_gemm): the gate/up pair is VALU-bound (the per-block
// f32 rescale), so occupancy hides more than ring depth there: 2 stages fit
// four gate/up workgroups per CU where 4 stages fit two (gate+up 104 -> 76 us
// at 512 tokens; 3 stages changed nothing). The narrow launches wait on
// their stage loads at 3 waves per SIMD and fill 4 stages, two at a time.

// WM = MFMA row tiles per wave: WM 2 gives waves of 32 rows x 16 tokens
// (workgroup 32 x 64), WM 1 waves of 16 rows x 16 tokens in a 2 x 2 grid
// (workgroup 32 x 32): twice the waves for the narrow projections, whose
// 32 x 64 grids leave SIMDs with one or two waves.
template <int WM>
constexpr int gemm_bn() { return WM == 2 ? 64 : 32; }
// The stage's scales are one contiguous run, filled by whole-wave 16-byte
// loads (one load per 256 floats, issued by waves 0 and 1): dw of the tile's
// 32 rows per block (gate, then up for the pair), then dx of its tokens per
// block. The narrow launches' stage time follows the count of load
// instructions more than their bytes, and two 8-lane scale loads per wave
// cost about as much as a full operand load.
template <bool GU, int WM>
struct GemmStageLds {
    static constexpr int SW = 0, SW2 = GK_BLK * GBM, SX = GK_BLK * GBM * (GU ? 2 : 1);
    static constexpr int NSC = SX + GK_BLK * gemm_bn<WM>();  // floats of scales
    static constexpr int SC_LOADS = (NSC + 255) / 256;       // wave loads of them (<= 2)
    int8_t a[GBM * 128];
    int8_t a2[GU ? GBM * 128 : 16];
    int8_t b[gemm_bn<WM>() * 128];
    float sc[NSC];
    __device__ __forceinline__ const float* sw() const { return sc + SW; }
    __device__ __forceinline__ const float* sw2() const { return sc + SW2; }
    __device__ __forceinline__ const float* sx() const { return sc + SX; }
};
typedef float v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void lds_load16(const void* g, void* lds_wave_base) { uq_lds_load16(g, lds_wave_base); }
// rows r and r+16 (read by one ds_read2 of the two MFMA row tiles) get different slots
__device__ __forceinline__ int swz(int row) { return ((row >> 1) ^ (row >> 4)) & 7; }

// Per-lane byte offsets of the stage loads from wave-uniform bases: each load
// is a uniform 64-bit base (scalar registers, advanced once per stage by
// scalar arithmetic) plus a 32-bit per-lane offset computed once, so the
// operand loads take the scalar-base addressing form and a stage costs no
// per-lane 64-bit address arithmetic. The offsets stay far below 2^32 (rows
// of the tile times K <= 16384, or scales of 4 blocks of rows n or tokens mp).
// Scale float f = 256 * wave + 4 * lane of the stage's run: gate dw, up dw
// (the pair) or dx, block f / 32 of the rows or f / BN of the tokens. Its
// source is the gate-scale cursor plus a per-lane byte offset `so` (flat
// addresses; the up and token scale planes are other allocations), which the
// token-scale lanes move by `sstep` per stage: the gate cursor advances
// 4 blocks of n floats, the token scales 4 blocks of mp. No per-lane pointer
// select (a select among the cursors became a table in scratch memory).
struct GemmSrc {
    uint32_t a, b0, b1;
    uint64_t so, sstep;
    bool sload;
};
template <bool GU, int WM>
__device__ __forceinline__ GemmSrc gemm_src(const PfGemmArgs& p, int64_t r0, int64_t t0, int wave, int lane) {
    typedef GemmStageLds<GU, WM> St;
    constexpr int BN = gemm_bn<WM>();
    const int K = (int)p.k;
    const int slot = lane & 7, row = 8 * wave + (lane >> 3);
    const int tk0 = 8 * WM * wave + (lane >> 3), tk1 = tk0 + 8;
    GemmSrc g;
    g.a = (uint32_t)(row * K + 16 * (slot ^ swz(row)));
    g.b0 = (uint32_t)(tk0 * K + 16 * (slot ^ swz(tk0)));
    g.b1 = (uint32_t)(tk1 * K + 16 * (slot ^ swz(tk1)));
    const int f = 256 * wave + 4 * lane;
    const uint64_t gate = (uint64_t)(p.w_ds + r0);
    g.sload = wave < St::SC_LOADS && f < St::NSC;
    g.so = 0;
    g.sstep = 0;
    if (f < St::SX) {
        const bool up = GU && f >= St::SW2;
        const int fw = up ? f - St::SW2 : f;
        const uint64_t seg = up ? (uint64_t)(p.w2_ds + r0) : gate;
        g.so = seg - gate + (uint64_t)(4 * ((fw / GBM) * p.n + fw % GBM));
    } else {
        const int fx = f - St::SX;
        g.so = (uint64_t)(p.xst + t0) - gate + (uint64_t)(4 * ((fx / BN) * (int64_t)p.mp + fx % BN));
        g.sstep = (uint64_t)(4 * GK_BLK * ((int64_t)p.mp - p.n));
    }
    return g;
}
__device__ __forceinline__ const void* at(const void* base, uint32_t off) {
    return (const char*)base + (uint64_t)off;
}

// Issue the global->LDS loads of one stage (first block kb) of the tile at
// rows r0, tokens t0. A partial last stage (nblk < 4) re-reads its last valid
// block in place of the missing ones (values unused).
template <bool GU, int WM>
__device__ __forceinline__ void gemm_issue(const PfGemmArgs& p, const GemmSrc& g, GemmStageLds<GU, WM>& S,
                                           int64_t r0, int64_t t0, int64_t kb, int nblk, int wave, int lane) {
    constexpr int BN = gemm_bn<WM>();
    const int slot = lane & 7;
    uint32_t oa = g.a, ob0 = g.b0, ob1 = g.b1;
    if (nblk < GK_BLK) {
        // chunk c = slot ^ swz(row) of block c/2; clamp the block, keep the half
        // (the shift is -32 * (blocks past the end) >= -(the chunk's own offset))
        const int row = 8 * wave + (lane >> 3), tk0 = 8 * WM * wave + (lane >> 3), tk1 = tk0 + 8;
        auto shift = [&](int r) {
            const int c = slot ^ swz(r), blk = c >> 1, cb = blk < nblk ? blk : nblk - 1;
            return (uint32_t)((cb - blk) * 32);
        };
        oa += shift(row);
        ob0 += shift(tk0);
        ob1 += shift(tk1);
    }
    const int64_t K = p.k, wa = r0 * K + kb * 32, wb = t0 * K + kb * 32;
    lds_load16(at(p.w_qs + wa, oa), S.a + wave * 1024);
    if (GU) lds_load16(at(p.w2_qs + wa, oa), S.a2 + wave * 1024);
    lds_load16(at(p.xq + wb, ob0), S.b + (WM * wave) * 1024);
    if (WM == 2) lds_load16(at(p.xq + wb, ob1), S.b + (2 * wave + 1) * 1024);
    typedef GemmStageLds<GU, WM> St;
    if (wave < St::SC_LOADS) {
        // the stage's scale run, blocks past the end clamped to the last one
        const int f = 256 * wave + 4 * lane;
        if (f < St::NSC) {
            const float* src;
            if (f < St::SX) {
                const bool up = GU && f >= St::SW2;
                const int fw = up ? f - St::SW2 : f, blk = fw / GBM < nblk ? fw / GBM : nblk - 1;
                src = (up ? p.w2_ds : p.w_ds) + (kb + blk) * p.n + r0 + fw % GBM;
            } else {
                const int fx = f - St::SX, blk = fx / BN < nblk ? fx / BN : nblk - 1;
                src = p.xst + (kb + blk) * (int64_t)p.mp + t0 + fx % BN;
            }
            lds_load16(src, S.sc + 256 * wave);
        }
    }
}


// Uniform source pointers of the next full stage (scalar registers), moved
// one stage (4 blocks) on with scalar adds; the per-lane offsets of GemmSrc
// are added at each load. Replaces the per-stage 64-bit products of the
// generic issue, which left each wave about as many scalar as vector
// instructions in the narrow launches.
template <bool GU>
struct GemmCursor {
    const int8_t* a;
    const int8_t* a2;
    const int8_t* b;
    const float* sw;  // gate scales of the stage's first block (the scale loads' base)
    __device__ __forceinline__ void advance(int64_t n) {
        a += GK_BLK * 32;
        b += GK_BLK * 32;
        sw += GK_BLK * n;
        if (GU) a2 += GK_BLK * 32;
    }
};

// The loads of the cursor's full stage (the same bytes gemm_issue loads for
// a stage of four blocks).
template <bool GU, int WM>
__device__ __forceinline__ void gemm_issue_full(const GemmCursor<GU>& c, const GemmSrc& g, GemmStageLds<GU, WM>& S,
                                                int wave, int lane) {
    constexpr int BN = gemm_bn<WM>();
    lds_load16(at(c.a, g.a), S.a + wave * 1024);
    if (GU) lds_load16(at(c.a2, g.a), S.a2 + wave * 1024);
    lds_load16(at(c.b, g.b0), S.b + (WM * wave) * 1024);
    if (WM == 2) lds_load16(at(c.b, g.b1), S.b + (2 * wave + 1) * 1024);
    if (wave < GemmStageLds<GU, WM>::SC_LOADS && g.sload)
        lds_load16((const void*)((uint64_t)c.sw + g.so), S.sc + 256 * wave);
}

// Wait until at most `n` vector-memory ops of this wave are outstanding
// (s_waitcnt vmcnt(n); expcnt and lgkmcnt left at their maxima).
template <int n>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14));
}

// Workgroup barrier without the release fence of __syncthreads: that fence
// waits for every outstanding vector-memory op, including the LDS-DMA loads
// of the later stages. Visibility of a stage is ensured by wait_vm before it;
// the empty asm statements keep the compiler from moving memory ops across.
__device__ __forceinline__ void stage_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads are done
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// NB consecutive 32-blocks (from j0) of a stage: every MFMA of the group is
// issued first, then the f32 rescale runs block by block in order.
template <bool GU, int WM, int NB>
__device__ __forceinline__ void gemm_blocks(const GemmStageLds<GU, WM>& S, int j0, int wc, int rb, int lane,
                                            float (&f)[WM][4], float (&g)[WM][4]) {
    constexpr int BN = gemm_bn<WM>();
    const int li = lane & 15, lm = (lane >> 4) * 4, sub = ((lane >> 4) & 1) * 8, hi = lane >> 5;
    const v4i z = {0, 0, 0, 0};
    v4i c[NB][WM], c2[NB][WM];
#pragma unroll
    for (int jj = 0; jj < NB; jj++) {
        const int j = j0 + jj, gc = 2 * j + hi;
        long av[WM], a2v[WM], bv;
#pragma unroll
        for (int m = 0; m < WM; m++) {
            const int row = rb + 16 * m + li;
            const int off = row * 128 + ((gc ^ swz(row)) << 4) + sub;
            av[m] = *(const long*)(S.a + off);
            if (GU) a2v[m] = *(const long*)(S.a2 + off);
        }
        {
            const int tok = wc + li;
            bv = *(const long*)(S.b + tok * 128 + ((gc ^ swz(tok)) << 4) + sub);
        }
#pragma unroll
        for (int m = 0; m < WM; m++) {
            c[jj][m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[m], bv, z, 0, 0, 0);
            if (GU) c2[jj][m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a2v[m], bv, z, 0, 0, 0);
        }
    }
    // Scale products dw[row][j] * dx[token][j] from v_mfma_f32_16x16x1f32:
    // four 16 x 16 outer products, the k-th in registers 4k..4k+3 at rows
    // 4*(lane/16) + q, token lane % 16 (the int8 MFMA's layout); lane l
    // supplies the k = l/16 product's row (A) and token (B) factor. Each
    // product is a single f32 multiply (round to nearest even, denormals
    // kept), the value w * x has on the VALU, which keeps a third of the
    // rescale off the VALU.
    typedef float v16f __attribute__((ext_vector_type(16)));
    const int kq = lane >> 4;
    if constexpr (GU) {
        // gate/up pair, one block per group (the live MFMA results and
        // products of two blocks would cost the fourth wave per SIMD):
        // product k = (gate k < 2 / up k >= 2) x (row tile k % 2)
        static_assert(NB == 1, "pair: one block per group");
        const int mk = (kq & 1) < WM ? (kq & 1) : 0;
        const float bx = S.sx()[j0 * BN + wc + li];
        const float* sws = kq >= 2 ? S.sw2() : S.sw();
        const float ax = sws[j0 * GBM + rb + 16 * mk + li];
        v16f z16;
#pragma unroll
        for (int r = 0; r < 16; r++) z16[r] = 0.0f;
        const v16f sc = __builtin_amdgcn_mfma_f32_16x16x1f32(ax, bx, z16, 0, 0, 0);
#pragma unroll
        for (int m = 0; m < WM; m++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                f[m][q] = fmaf((float)c[0][m][q], sc[4 * m + q], f[m][q]);
                g[m][q] = fmaf((float)c2[0][m][q], sc[4 * (2 + m) + q], g[m][q]);
            }
    } else {
        // one product per block of the group's 4, per row tile
        static_assert(NB == 4, "one outer-product MFMA per group and row tile");
        const float bx = S.sx()[(j0 + kq) * BN + wc + li];
        v16f sc[WM];
#pragma unroll
        for (int m = 0; m < WM; m++) {
            const float ax = S.sw()[(j0 + kq) * GBM + rb + 16 * m + li];
            v16f z16;
#pragma unroll
            for (int r = 0; r < 16; r++) z16[r] = 0.0f;
            sc[m] = __builtin_amdgcn_mfma_f32_16x16x1f32(ax, bx, z16, 0, 0, 0);
        }
#pragma unroll
        for (int jj = 0; jj < NB; jj++)
#pragma unroll
            for (int m = 0; m < WM; m++)
#pragma unroll
                for (int q = 0; q < 4; q++) f[m][q] = fmaf((float)c[jj][m][q], sc[m][4 * jj + q], f[m][q]);
    }
}

// One 32-block (a partial last stage): MFMA, then the rescale with the scale
// product on the VALU.
template <bool GU, int WM>
__device__ __forceinline__ void gemm_block_tail(const GemmStageLds<GU, WM>& S, int j, int wc, int rb, int lane,
                                                float (&f)[WM][4], float (&g)[WM][4]) {
    constexpr int BN = gemm_bn<WM>();
    const int li = lane & 15, lm = (lane >> 4) * 4, sub = ((lane >> 4) & 1) * 8, hi = lane >> 5;
    const v4i z = {0, 0, 0, 0};
    const int gc = 2 * j + hi, tok = wc + li;
    const long bv = *(const long*)(S.b + tok * 128 + ((gc ^ swz(tok)) << 4) + sub);
    const float x = S.sx()[j * BN + wc + li];
#pragma unroll
    for (int m = 0; m < WM; m++) {
        const int row = rb + 16 * m + li;
        const int off = row * 128 + ((gc ^ swz(row)) << 4) + sub;
        const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(*(const long*)(S.a + off), bv, z, 0, 0, 0);
        v4i c2;
        if (GU) c2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(*(const long*)(S.a2 + off), bv, z, 0, 0, 0);
        const v4f w = *(const v4f*)(S.sw() + j * GBM + rb + 16 * m + lm);
        v4f w2;
        if (GU) w2 = *(const v4f*)(S.sw2() + j * GBM + rb + 16 * m + lm);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            f[m][q] = fmaf((float)c[q], w[q] * x, f[m][q]);
            if (GU) g[m][q] = fmaf((float)c2[q], w2[q] * x, g[m][q]);
        }
    }
}

// The q|k|v launch's epilogue (PfRopeEpi): a lane's 4 consecutive permuted
// rows r..r+3 of token t are two RoPE pairs (outputs j, j + hd/2 and j + 1,
// j + 1 + hd/2 of one head) or 4 v values. Per pair, as prefill_rope
// (gpu_prefill.cu:73-81): u = x + bias, w = x' + bias', then u*cos - w*sin and
// u*sin + w*cos with each product rounded, q kept f32, k and v rounded to fp16.
__device__ __forceinline__ void rope_store(const PfRopeEpi& e, int64_t t, int r, const float (&v)[4]) {
    if (t >= e.n) return;  // padding tokens: no cache row past the prompt is written
    const int hd = e.head_dim, half = hd / 2, dim = e.heads * hd, kvd = e.kv_heads * hd;
    const int pos = e.p0 + (int)t;
    const float4 b4 = *(const float4*)(e.bias + r);
    const float bx[4] = {b4.x, b4.y, b4.z, b4.w};
    if (r < dim + kvd) {
        const bool isq = r < dim, hb = isq ? e.hb_q != 0 : e.hb_k != 0;
        const int w0 = isq ? r : r - dim, h = w0 / hd, j = (w0 % hd) / 2;
        const float* tr = e.trig + (size_t)pos * hd;
        const float2 cc = *(const float2*)(tr + j), ss = *(const float2*)(tr + half + j);
        const float c0[2] = {cc.x, cc.y}, c1[2] = {ss.x, ss.y};
        float ra[2], rb[2];
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const float uu = hb ? v[2 * p] + bx[2 * p] : v[2 * p];
            const float ww = hb ? v[2 * p + 1] + bx[2 * p + 1] : v[2 * p + 1];
            const float p0 = uu * c0[p], p1 = ww * c1[p], p2 = uu * c1[p], p3 = ww * c0[p];
            ra[p] = p0 - p1;
            rb[p] = p2 + p3;
        }
        const int ia = h * hd + j, ib = ia + half;
        if (isq) {
            float* qr = e.q + t * e.stride;
            *(float2*)(qr + ia) = make_float2(ra[0], ra[1]);
            *(float2*)(qr + ib) = make_float2(rb[0], rb[1]);
        } else {
            uint16_t* kr = e.kcache + (size_t)pos * kvd;
            *(uint32_t*)(kr + ia) = uq_f16_rne(ra[0]) | (uint32_t)uq_f16_rne(ra[1]) << 16;
            *(uint32_t*)(kr + ib) = uq_f16_rne(rb[0]) | (uint32_t)uq_f16_rne(rb[1]) << 16;
        }
    } else {
        const int e0 = r - dim - kvd;
        uint16_t hv[4];
#pragma unroll
        for (int m = 0; m < 4; m++) hv[m] = uq_f16_rne(e.hb_v ? v[m] + bx[m] : v[m]);
        *(uint2*)(e.vcache + (size_t)pos * kvd + e0) =
            make_uint2(hv[0] | (uint32_t)hv[1] << 16, hv[2] | (uint32_t)hv[3] << 16);
    }
}

template <bool GU, int WM>
__global__ __launch_bounds__(256) void k_pf_gemm(PfGemmArgs a) {
    // ring stages: the gate/up pair and the wide tiles fill two, one ahead
    // (four would halve their workgroups per CU); the narrow launches (WM 1)
    // fill four, two at a time, with one wait and barrier per pair of stages
    constexpr int RG = GU || WM == 2 ? 2 : 4;
    __shared__ __attribute__((aligned(16))) GemmStageLds<GU, WM> ring[RG];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // the wave's tile: tokens wc.. of the workgroup's, rows rb..
    const int wc = WM == 2 ? wave * 16 : (wave >> 1) * 16, rb = WM == 2 ? 0 : (wave & 1) * 16;
    const int64_t r0 = (int64_t)blockIdx.x * GBM, t0 = (int64_t)blockIdx.y * gemm_bn<WM>();
    // k <= 16384: at most 512 blocks, 128 stages
    const int nb = (int)(a.k / 32), nst = (nb + GK_BLK - 1) / GK_BLK, nfull = nb / GK_BLK;
    auto nblk_of = [&](int s) { return nb - s * GK_BLK < GK_BLK ? nb - s * GK_BLK : GK_BLK; };
    float f[WM][4], g[WM][4];
#pragma unroll
    for (int m = 0; m < WM; m++)
#pragma unroll
        for (int q = 0; q < 4; q++) f[m][q] = g[m][q] = 0.0f;
    GemmSrc src = gemm_src<GU, WM>(a, r0, t0, wave, lane);
    GemmCursor<GU> cur{a.w_qs + r0 * a.k, GU ? a.w2_qs + r0 * a.k : nullptr, a.xq + t0 * a.k, a.w_ds + r0};
    // stage s's loads, issued in stage order: full stages from the cursor, a
    // partial last stage through the clamping issue
    auto issue = [&](int s) {
        GemmStageLds<GU, WM>& S = ring[s & (RG - 1)];
        if (s < nfull) {
            gemm_issue_full<GU, WM>(cur, src, S, wave, lane);
            cur.advance(a.n);
            src.so += src.sstep;
        } else {
            gemm_issue<GU, WM>(a, src, S, r0, t0, (int64_t)s * GK_BLK, nblk_of(s), wave, lane);
        }
    };
    auto compute = [&](int s) {
        const GemmStageLds<GU, WM>& S = ring[s & (RG - 1)];
        if (s < nfull) {
            if constexpr (GU) {
#pragma unroll
                for (int j = 0; j < GK_BLK; j++) gemm_blocks<GU, WM, 1>(S, j, wc, rb, lane, f, g);
            } else {
                gemm_blocks<GU, WM, GK_BLK>(S, 0, wc, rb, lane, f, g);
            }
        } else {
            const int nblk = nblk_of(s);
            for (int j = 0; j < nblk; j++) gemm_block_tail<GU, WM>(S, j, wc, rb, lane, f, g);
        }
    };
    // Each step: this wave's loads of the step's stages landed (nothing later
    // is in flight), then the barrier makes every wave's loads visible and
    // frees the ring slots the next loads fill. Full steps run in a loop with
    // no other path, so the accumulators stay in their registers.
    constexpr int STEP = RG / 2;
    for (int s = 0; s < STEP && s < nst; s++) issue(s);
    int s = 0;
    for (; s + STEP <= nfull; s += STEP) {
        wait_vm<0>();
        stage_barrier();
#pragma unroll
        for (int u = STEP; u < 2 * STEP; u++)
            if (s + u < nst) issue(s + u);
#pragma unroll
        for (int u = 0; u < STEP; u++) {
            // the pair block by block, the others as one group of 4
            if constexpr (GU) {
#pragma unroll
                for (int j = 0; j < GK_BLK; j++) gemm_blocks<GU, WM, 1>(ring[(s + u) & (RG - 1)], j, wc, rb, lane, f, g);
            } else {
                gemm_blocks<GU, WM, GK_BLK>(ring[(s + u) & (RG - 1)], 0, wc, rb, lane, f, g);
            }
        }
    }
    if (s < nst) {
        // fewer than STEP full stages and / or the partial stage remain, all issued
        wait_vm<0>();
        stage_barrier();
        for (int u = s; u < nst; u++) compute(u);
    }
    const int li = lane & 15, lm = (lane >> 4) * 4;
    if (GU && WM == 2 && a.yq) {
        // SiLU(gate)*up quantized per 32-block into the next GEMM's planes:
        // the workgroup's 32 rows are one block of each token, held by lanes
        // li, li+16, li+32, li+48 (8 values each) of one wave
        float o[WM][4];
        float am = 0.0f;
#pragma unroll
        for (int m = 0; m < WM; m++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                o[m][q] = uq_silu_mul(f[m][q], g[m][q]);
                am = (m | q) ? fmaxf(am, fabsf(o[m][q])) : fabsf(o[m][q]);
            }
        am = fmaxf(am, __shfl_xor(am, 16, 64));
        am = fmaxf(am, __shfl_xor(am, 32, 64));
        const float inv = am > 0.0f ? 127.0f / am : 0.0f;
        const int64_t t = t0 + wc + li;
#pragma unroll
        for (int m = 0; m < WM; m++) {
            uint32_t p = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) p |= uq_quant_code(o[m][q], inv) << (8 * q);
            *(uint32_t*)(a.yq + t * a.n + r0 + 16 * m + lm) = p;
        }
        if (lane < 16) a.yst[(r0 / 32) * a.mp + t] = am / 127.0f;
        return;
    }
#pragma unroll
    for (int m = 0; m < WM; m++) {
        const int64_t t = t0 + wc + li, r = r0 + rb + 16 * m + lm;
        if (!GU && a.rope) {
            rope_store(a.re, t, (int)r, f[m]);
            continue;
        }
        float4 o;
        if (GU) {
            o = make_float4(uq_silu_mul(f[m][0], g[m][0]), uq_silu_mul(f[m][1], g[m][1]),
                            uq_silu_mul(f[m][2], g[m][2]), uq_silu_mul(f[m][3], g[m][3]));
        } else {
            o = make_float4(f[m][0], f[m][1], f[m][2], f[m][3]);
        }
        *(float4*)(a.y + t * a.n + r) = o;
    }
}

// ------------------------------------------------------------------ row gathers
// The prefill copy of the q|k|v weight with the RoPE partners adjacent
// (PfRopeEpi): dst row r = src row perm[r], 16 bytes per thread.
__global__ __launch_bounds__(256) void k_gather_rows(const int8_t* __restrict__ src, int64_t rowb,
                                                     const int* __restrict__ perm, int64_t m, int8_t* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x, per = rowb / 16;
    if (i >= m * per) return;
    const int64_t r = i / per, c = i % per;
    ((int4*)(dst + r * rowb))[c] = ((const int4*)(src + (int64_t)perm[r] * rowb))[c];
}
// dst[b][r] = src[b][perm[r]] on [nb][m] planes (the transposed scales, the bias)
__global__ __launch_bounds__(256) void k_gather_cols(const float* __restrict__ src, int64_t nb, int64_t m,
                                                     const int* __restrict__ perm, float* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nb * m) return;
    const int64_t b = i / m, r = i % m;
    dst[i] = src[b * m + perm[r]];
}

// ------------------------------------------------------------------ causal attention
// Workgroup = (query head, tile of 16 consecutive queries), 4 waves. Same
// arithmetic as decode attention: q.k in double (each product f32 x fp16 is
// exact in double), * 1/sqrt(hd) in f32, max-subtracted exp, total in double,
// p = e/total, P.V in double. Both contractions run on the FP64 MFMA
// v_mfma_f64_16x16x4_f64 (D += A B, A 16x4, B 4x16): lane l holds A[l%16][l/16]
// and B[l/16][l%16], and register r of lane l holds D[4r + l/16][l%16].
//   q.k: A = Q (16 queries x 4 dims), B = K^T (4 dims x 16 keys); lane group
//        g = l/16 takes dims [g*HD/4, (g+1)*HD/4), one per MFMA step, so each
//        lane's q and k pieces are contiguous. Waves take key tiles of 16 in turn.
//   P.V: A = P (16 queries x 4 keys) from LDS, B = V (4 keys x 16 dims); each
//        wave owns HD/64 tiles of 16 dims.
// The double sums run in MFMA order instead of the oracle's sequential order;
// every term is exact, so the f32 results agree except when a double sum
// lands within an ulp of an f32 rounding boundary.
constexpr int PA_Q = 16;
template <int HD>
__global__ __launch_bounds__(256) void k_pf_attention(PfAttnArgs a) {
    extern __shared__ float ps[];  // [PA_Q][sst]: scores, then p (0 past each query's causal end)
    constexpr int DG = HD / 4;     // dims per lane group in q.k
    constexpr int DT = HD / 64;    // 16-dim tiles per wave in P.V
    typedef double d4 __attribute__((ext_vector_type(4)));
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, c = lane & 15;
    // Work rank r orders the (tile, head) pairs by descending key count. The
    // first ncu workgroup ids take ranks 0.. (longest first, one per CU); the
    // remaining ids take the shortest ranks first, so a CU's second resident
    // workgroup is short where its first is long (the longest tile sets the
    // kernel's duration: 2,048 FP64 MFMAs on the CU's four SIMDs)
    const int L = blockIdx.y * gridDim.x + blockIdx.x, total = gridDim.x * gridDim.y;
    const int r = L < a.ncu ? L : total - 1 - (L - a.ncu);
    const int h = r % gridDim.x, kh = h / (a.heads / a.kv_heads), kvd = a.kv_heads * HD;
    const int tq0 = (gridDim.y - 1 - r / gridDim.x) * PA_Q;
    const int nq = a.n - tq0 < PA_Q ? a.n - tq0 : PA_Q;  // live queries of the tile
    const int sst = (a.p0 + a.n + 15) & ~15;              // LDS row stride (keys)
    const int kend = a.p0 + tq0 + nq;                     // keys needed by the tile: [0, kend)
    const int kpad = (kend + 3) & ~3;                     // P.V runs over whole 4-key steps
    // q operand: query c of the tile, dims [g*DG, (g+1)*DG) as doubles
    double qa[DG];
    {
        const bool qlive = c < nq;
        const float* qr = a.qkv + (size_t)(tq0 + (qlive ? c : 0)) * a.stride + h * HD + g * DG;
#pragma unroll
        for (int i = 0; i < DG; i += 4) {
            const float4 v = *(const float4*)(qr + i);
            qa[i] = qlive ? (double)v.x : 0.0;
            qa[i + 1] = qlive ? (double)v.y : 0.0;
            qa[i + 2] = qlive ? (double)v.z : 0.0;
            qa[i + 3] = qlive ? (double)v.w : 0.0;
        }
    }
    // scores of key tiles kt = wave, wave + 4, ...; the next tile's K is
    // loaded before the current tile's MFMAs
    const int ntile = (kend + 15) >> 4;
    auto load_k = [&](int kt, uint32_t* kw) {
        // keys past the tile's causal end are read from key kend-1 (written,
        // in bounds) and their scores are never used
        int key = kt * 16 + c;
        key = key < kend ? key : kend - 1;
        const uint16_t* kr = a.kcache + (size_t)key * kvd + kh * HD + g * DG;
#pragma unroll
        for (int i = 0; i < DG / 8; i++) {
            const int4 v = *(const int4*)(kr + 8 * i);
            kw[4 * i] = (uint32_t)v.x;
            kw[4 * i + 1] = (uint32_t)v.y;
            kw[4 * i + 2] = (uint32_t)v.z;
            kw[4 * i + 3] = (uint32_t)v.w;
        }
    };
    // four independent accumulator chains (steps i mod 4), summed at the end;
    // the B operands of 16 MFMAs are converted to double into their own
    // registers first, then the 16 MFMAs issue back to back (converted one by
    // one into a reused register, each MFMA waited on its conversion:
    // prefill 5.74 -> 5.67 ms)
    auto score_tile = [&](int kt, const uint32_t* kw) {
        d4 acc[4];
#pragma unroll
        for (int k = 0; k < 4; k++) acc[k] = d4{0.0, 0.0, 0.0, 0.0};
        constexpr int HB = DG < 16 ? DG : 16;
#pragma unroll
        for (int i0 = 0; i0 < DG; i0 += HB) {
            double kd[HB];
#pragma unroll
            for (int i = 0; i < HB; i++) {
                const int ii = i0 + i;
                const uint16_t hk = (uint16_t)(ii & 1 ? kw[ii >> 1] >> 16 : kw[ii >> 1] & 0xffff);
                kd[i] = (double)uq_half(hk);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < HB; i++)
                acc[(i0 + i) & 3] = __builtin_amdgcn_mfma_f64_16x16x4f64(qa[i0 + i], kd[i], acc[(i0 + i) & 3], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        const d4 sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
#pragma unroll
        for (int r = 0; r < 4; r++) ps[(4 * r + g) * sst + kt * 16 + c] = (float)sum[r] * a.qscale;
    };
    {
        uint32_t ka[DG / 2], kb[DG / 2];
        int kt = wave;
        if (kt < ntile) load_k(kt, ka);
        // sched_barrier: the scheduler would otherwise sink the prefetch below the MFMAs
        while (kt < ntile) {
            if (kt + 4 < ntile) load_k(kt + 4, kb);
            __builtin_amdgcn_sched_barrier(0);
            score_tile(kt, ka);
            kt += 4;
            if (kt >= ntile) break;
            if (kt + 4 < ntile) load_k(kt + 4, ka);
            __builtin_amdgcn_sched_barrier(0);
            score_tile(kt, kb);
            kt += 4;
        }
    }
    __syncthreads();
    // softmax: 16 lanes per query (query tid/16 of the tile), 4 consecutive
    // keys per lane per LDS read; keys past the causal end become p = 0
    {
        const int qi = tid >> 4, cj = tid & 15;
        const int T = qi < nq ? a.p0 + tq0 + qi + 1 : 0;  // causal: keys [0, T)
        float* sr = ps + qi * sst;
        float mx = -3.402823466e38f;
        for (int t0 = 4 * cj; t0 < T; t0 += 64) {
            const float4 v = *(const float4*)(sr + t0);
            mx = fmaxf(mx, v.x);
            if (t0 + 1 < T) mx = fmaxf(mx, v.y);
            if (t0 + 2 < T) mx = fmaxf(mx, v.z);
            if (t0 + 3 < T) mx = fmaxf(mx, v.w);
        }
        mx = uq_group_max<16>(mx);
        double tot = 0.0;
        // every score read is finite (keys past T hold later queries' or the
        // clamped key's scores), so all four exps run and the masked ones
        // become 0 by select: no divergent branch per key
        for (int t0 = 4 * cj; t0 < T; t0 += 64) {
            const float4 v = *(const float4*)(sr + t0);
            const float e0 = uq_expf(v.x - mx);
            float e1 = uq_expf(v.y - mx), e2 = uq_expf(v.z - mx), e3 = uq_expf(v.w - mx);
            e1 = t0 + 1 < T ? e1 : 0.0f;
            e2 = t0 + 2 < T ? e2 : 0.0f;
            e3 = t0 + 3 < T ? e3 : 0.0f;
            *(float4*)(sr + t0) = make_float4(e0, e1, e2, e3);
            tot += (double)e0;
            tot += (double)e1;
            tot += (double)e2;
            tot += (double)e3;
        }
        tot = uq_group_sum<16>(tot);
        const float total = (float)tot;
        for (int t0 = 4 * cj; t0 < kpad; t0 += 64) {
            const float4 v = *(const float4*)(sr + t0);
            const float p0 = t0 < T ? v.x / total : 0.0f;
            const float p1 = t0 + 1 < T ? v.y / total : 0.0f;
            const float p2 = t0 + 2 < T ? v.z / total : 0.0f;
            const float p3 = t0 + 3 < T ? v.w / total : 0.0f;
            *(float4*)(sr + t0) = make_float4(p0, p1, p2, p3);
        }
    }
    __syncthreads();
    // P.V: this wave's dim tiles d0 = (wave * DT + j) * 16
    d4 o[DT];
#pragma unroll
    for (int j = 0; j < DT; j++) o[j] = d4{0.0, 0.0, 0.0, 0.0};
    const float* pr = ps + c * sst;  // A row: query c
    const uint16_t* vb = a.vcache + kh * HD + wave * DT * 16 + c;
    // batches of SU 4-key steps in a two-stage register pipeline: the next
    // batch's P and V loads are issued before the current batch's MFMAs
    constexpr int SU = 8;
    // p stays f32 (and unmasked) until the batch's MFMAs: the LDS reads and V
    // loads of a batch issue back to back with no per-key wait or branch
    struct PvBatch { float p[SU]; uint16_t v[SU][DT]; };
    auto load_pv = [&](int k0, PvBatch& bt) {
#pragma unroll
        for (int u = 0; u < SU; u++) {
            const int kk = k0 + 4 * u + g;
            const int kl = kk < kpad ? kk : kpad - 1;
            const int kv = kl < kend ? kl : kend - 1;  // p is 0 there
            bt.p[u] = pr[kl];
#pragma unroll
            for (int j = 0; j < DT; j++) bt.v[u][j] = vb[(size_t)kv * kvd + j * 16];
        }
    };
    // two accumulator chains per dim tile (even and odd steps), summed at the end
    d4 o2[DT];
#pragma unroll
    for (int j = 0; j < DT; j++) o2[j] = d4{0.0, 0.0, 0.0, 0.0};
    // the batch's V operands converted to double first, then its MFMAs
    // k0: the batch's first key; steps past kpad get p = 0
    auto mma_pv = [&](int k0, const PvBatch& bt) {
        double vd[SU][DT], pd[SU];
#pragma unroll
        for (int u = 0; u < SU; u++) {
            pd[u] = k0 + 4 * u + g < kpad ? (double)bt.p[u] : 0.0;
#pragma unroll
            for (int j = 0; j < DT; j++) vd[u][j] = (double)uq_half(bt.v[u][j]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < SU; u += 2)
#pragma unroll
            for (int j = 0; j < DT; j++) {
                o[j] = __builtin_amdgcn_mfma_f64_16x16x4f64(pd[u], vd[u][j], o[j], 0, 0, 0);
                o2[j] = __builtin_amdgcn_mfma_f64_16x16x4f64(pd[u + 1], vd[u + 1][j], o2[j], 0, 0, 0);
            }
        __builtin_amdgcn_sched_barrier(0);
    };
    {
        PvBatch ba, bb;
        int k0 = 0;
        if (k0 < kpad) load_pv(k0, ba);
        while (k0 < kpad) {
            if (k0 + 4 * SU < kpad) load_pv(k0 + 4 * SU, bb);
            __builtin_amdgcn_sched_barrier(0);
            mma_pv(k0, ba);
            k0 += 4 * SU;
            if (k0 >= kpad) break;
            if (k0 + 4 * SU < kpad) load_pv(k0 + 4 * SU, ba);
            __builtin_amdgcn_sched_barrier(0);
            mma_pv(k0, bb);
            k0 += 4 * SU;
        }
    }
    if (DT * 16 == 32 && a.xq) {
        // this wave's 32 dims of head h are one quant block of each query: the
        // block's values sit in the 16 lanes of group g (DT each)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int qi = 4 * r + g;
            float v[DT];
            float am = 0.0f;
#pragma unroll
            for (int j = 0; j < DT; j++) {
                v[j] = (float)(o[j][r] + o2[j][r]);
                am = j ? fmaxf(am, fabsf(v[j])) : fabsf(v[j]);
            }
            am = uq_group_max<16>(am);
            const float inv = am > 0.0f ? 127.0f / am : 0.0f;
            if (qi < nq) {
                const size_t col = (size_t)h * HD + wave * DT * 16;
                int8_t* q = a.xq + (size_t)(tq0 + qi) * (a.heads * HD) + col + c;
#pragma unroll
                for (int j = 0; j < DT; j++) q[j * 16] = (int8_t)uq_quant_code(v[j], inv);
                if (c == 0) a.xst[(col / 32) * a.mp + tq0 + qi] = am / 127.0f;
            }
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int qi = 4 * r + g;
        if (qi < nq) {
            float* out = a.out + (size_t)(tq0 + qi) * (a.heads * HD) + h * HD + wave * DT * 16 + c;
#pragma unroll
            for (int j = 0; j < DT; j++) out[j * 16] = (float)(o[j][r] + o2[j][r]);
        }
    }
}

}  // namespace

void launch_transpose_scales(const uint16_t* d, int64_t rows, int64_t nb, float* dt, hipStream_t s) {
    hipLaunchKernelGGL(k_transpose_scales, dim3((unsigned)((rows * nb + 255) / 256)), dim3(256), 0, s, d, rows, nb, dt);
}
template <int NC>
void pf_norm_nc(const PfNormArgs& a, int tokens, hipStream_t s) {
    if constexpr (NC > 1) {
        if (a.nq.dim / 256 < NC) return pf_norm_nc<NC - 1>(a, tokens, s);
    }
    hipLaunchKernelGGL(k_pf_norm<NC>, dim3(tokens), dim3(64 * NC), 0, s, a);
}
void launch_pf_norm(const PfNormArgs& a, int tokens, hipStream_t s) {
    // dim % 256 == 0 and dim <= PF_MAXD (checked at model creation)
    pf_norm_nc<PF_MAXD / 256>(a, tokens, s);
}
void launch_pf_quant(const float* x, int64_t k, int tokens, int mp, int8_t* xq, float* xst, hipStream_t s) {
    hipLaunchKernelGGL(k_pf_quant, dim3((unsigned)((k + 255) / 256), tokens), dim3(256), 0, s, x, k, mp, xq, xst);
}
int launch_pf_gemm(const PfGemmArgs& a, hipStream_t s) {
    if (a.n % 64 || a.mp % 64 || a.k % 32 || a.k <= 0) return -1;
    // 32 x 64 workgroup tiles unless that grid gives fewer than four
    // workgroups per CU; then 32 x 32 tiles of 16 x 16 waves
    if (a.yq && (!a.w2_qs || !a.yst)) return -1;
    // the quantizing gate/up epilogue needs a wave's tile to hold whole blocks (wide tiles)
    const bool narrow = !a.yq && (a.n / GBM) * (a.mp / 64) < 4 * (int64_t)cu_count();
    if (narrow) {
        const dim3 grid((unsigned)(a.n / GBM), (unsigned)(a.mp / gemm_bn<1>()));
        if (a.w2_qs) hipLaunchKernelGGL((k_pf_gemm<true, 1>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((k_pf_gemm<false, 1>), grid, dim3(256), 0, s, a);
    } else {
        const dim3 grid((unsigned)(a.n / GBM), (unsigned)(a.mp / gemm_bn<2>()));
        if (a.w2_qs) hipLaunchKernelGGL((k_pf_gemm<true, 2>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((k_pf_gemm<false, 2>), grid, dim3(256), 0, s, a);
    }
    return 0;
}
void launch_gather_rows(const int8_t* src, int64_t rowb, const int* perm, int64_t m, int8_t* dst, hipStream_t s) {
    const int64_t n = m * (rowb / 16);
    hipLaunchKernelGGL(k_gather_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, rowb, perm, m, dst);
}
void launch_gather_cols(const float* src, int64_t nb, int64_t m, const int* perm, float* dst, hipStream_t s) {
    hipLaunchKernelGGL(k_gather_cols, dim3((unsigned)((nb * m + 255) / 256)), dim3(256), 0, s, src, nb, m, perm, dst);
}
int launch_pf_attention(const PfAttnArgs& a0, hipStream_t s) {
    PfAttnArgs a = a0;
    a.ncu = cu_count();
    const size_t sst = (size_t)((a.p0 + a.n + 15) & ~15);
    const size_t lds = sizeof(float) * PA_Q * sst;
    if (lds > 65536 || a.n <= 0 || a.p0 + a.n > a.kcap || a.heads % a.kv_heads) return -1;
    const dim3 grid(a.heads, (a.n + PA_Q - 1) / PA_Q);
    switch (a.head_dim) {
    case 64: hipLaunchKernelGGL(k_pf_attention<64>, grid, dim3(256), lds, s, a); return 0;
    case 128: hipLaunchKernelGGL(k_pf_attention<128>, grid, dim3(256), lds, s, a); return 0;
    default: return -1;
    }
}

}  // namespace uq
