// Fused decode-step kernels for gfx950.
//
// Per transformer layer:
//   qkv_rope   residual + RMSNorm + quant prologue, q|k|v matvec, q/k bias,
//              RoPE, fp16 K/V store at `pos` (fused_resnorm + quant_act +
//              qkv_dp4a + rope_bias: gpu_fused.cu:28-35, gpu_dp4a.cu:23-59,
//              gpu_ops.cu:9-20)
//   attention  GQA softmax attention over the fp16 cache split over position
//              chunks: scores, then P.V into a double accumulator
//              (fused_attention, gpu_attention.cu:2-26)
//   o matvec   accumulator -> f32 -> block-32 quant prologue, Q8_0 matvec
//              (quant_act + linear_dp4a)
//   gateup_q   residual + RMSNorm + quant prologue, gate/up matvec, SiLU*up,
//              block-32 quant (gateup_dp4a, gpu_dp4a.cu:60-64)
//   down       generic matvec
// and per token: output RMSNorm, lm_head matvec with per-workgroup argmax,
// greedy finish (greedy_tiles / greedy_finish, gpu_greedy.cu:1-27).
//
// Fusion runs forward: a consumer workgroup recomputes the residual sum and
// RMSNorm of the 1536-wide activation itself (from L2) while its weight loads
// are in flight, instead of a producer workgroup publishing it. On this chip a
// device-scope fence inside a kernel writes back the XCD's L2, so producer
// "last workgroup" tails cost more than they save. The summed residual is
// stored by workgroup 0 into the other buffer of a ping-pong pair.
#include "uq_device.h"
#include "uq_units.h"
#include "uq_blockops.h"
#include "uq_step.h"
#include "uq_internal.h"

namespace uq {
namespace {

constexpr int MAX_DIM = 4096;

// ------------------------------------------------------------------ qkv + rope
// One wave per row pair (32 lanes per row): pair (j, j+hd/2) of a q or k head
// is rotated together; v rows are paired the same way and stored unrotated.
template <int NBL>
__global__ __launch_bounds__(320) void k_qkv_rope(QkvArgs a) {
    constexpr int NC = 2 * NBL < MAX_DIM / 256 ? 2 * NBL : MAX_DIM / 256;  // dim <= 32 lanes x NBL units x 16
    __shared__ __attribute__((aligned(16))) int8_t sq[NC * 256];
    __shared__ float ssc[NC * 8];
    __shared__ double part[5];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane & 31, grp = lane >> 5;
    const int hd = a.head_dim, half = hd / 2, kvd = a.kv_heads * hd;
    const int nq = a.heads * half, nk = a.kv_heads * half, npairs = nq + 2 * nk;
    // waves 0..3 hold one row pair each; wave 4 (and a wave past the last
    // pair) repeats the loads of the workgroup's first pair -- the same cache
    // lines -- so that every wave issues the same loads with no branch, which
    // keeps the waits of the prologue below exact
    const int pw = blockIdx.x * 4 + (wave < 4 ? wave : 0);
    const bool live = wave < 4 && pw < npairs;
    const int pu = pw < npairs ? pw : npairs - 1;
    const int region = pu < nq ? 0 : (pu < nq + nk ? 1 : 2);
    const int p = region == 0 ? pu : (region == 1 ? pu - nq : pu - nq - nk);
    const int h = p / half, j = p % half;
    const int ia = h * hd + j, ib = ia + half;  // within the region
    const int rbase = region == 0 ? 0 : (region == 1 ? a.heads * hd : a.heads * hd + kvd);
    const int64_t nu = a.dim / Q8::UNIT;
    const WArgs w{a.w_qs, a.w_d, nullptr};
    // The residual + RMSNorm + quant of the input is shared by all five waves
    // (the weight stream of this kernel is short): each wave loads its chunks
    // first, then the position (scalar read), its pair's bias and RoPE
    // operands and its weights, then normalizes and quantizes its chunks while
    // those loads are in flight.
    NormQuantSplit<NC, 5> nw;
    nw.issue(a.nq);
    const int pos = uq_sload(a.pos);
    // without a bias the two loads read the RoPE table instead (never used)
    const float* bias = region == 0 ? a.bq : (region == 1 ? a.bk : a.bv);
    const float ba = *(bias ? bias + ia : a.trig), bb = *(bias ? bias + ib : a.trig);
    const float cs = a.trig[(size_t)pos * hd + j];
    const float sn = a.trig[(size_t)pos * hd + half + j];
    Q8::W wv[NBL];
    {
        const Q8::R r = Q8::row_ptr(w, rbase + (grp ? ib : ia), nu);
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int u = sub + 32 * i, uc = u < nu ? u : (int)nu - 1;
            wv[i] = Q8::load_u(r, uc);
        }
    }
    nw.finish(a.nq, blockIdx.x == 0, part, sq, ssc);
    __syncthreads();    // the quantized input in LDS
    if (!live) return;  // whole wave; no barrier follows
    double acc = 0.0;  // never -0.0, so adding +0.0 for a clamped unit leaves it unchanged
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + 32 * i, uc = u < nu ? u : (int)nu - 1;
        Q8::X x;
        x.a = *(const int4*)(sq + 16 * uc);
        x.s = ssc[uc >> 1];
        const double t = Q8::dot(wv[i], x);
        acc += u < nu ? t : 0.0;
    }
    const float y = (float)uq_group_sum<32>(acc);
    const float yb = __shfl(y, 32, 64);
    if (lane != 0) return;
    const bool has_bias = region == 0 ? a.bq != nullptr : (region == 1 ? a.bk != nullptr : a.bv != nullptr);
    if (region == 2) {
        const float va = has_bias ? y + ba : y;
        const float vb = has_bias ? yb + bb : yb;
        a.vcache[(size_t)pos * kvd + ia] = uq_f16_rne(va);
        a.vcache[(size_t)pos * kvd + ib] = uq_f16_rne(vb);
        return;
    }
    const float u = has_bias ? y + ba : y;
    const float v = has_bias ? yb + bb : yb;
    const float p0 = u * cs, p1 = v * sn, p2 = u * sn, p3 = v * cs;
    const float ra = p0 - p1, rb = p2 + p3;
    if (region == 0) {
        a.q[ia] = ra;
        a.q[ib] = rb;
    } else {
        a.kcache[(size_t)pos * kvd + ia] = uq_f16_rne(ra);
        a.kcache[(size_t)pos * kvd + ib] = uq_f16_rne(rb);
    }
}

// ------------------------------------------------------------------ split attention
// Scores: workgroup (head, chunk) covers positions [lo, hi) of the chunk with
// HD/8 lanes per position (8 dims each, one 16-byte fp16 load), AS_B
// positions per lane in flight. q.k in double, butterfly over the position's
// lanes, * 1/sqrt(hd), rounded to f32 -- the oracle's score bits.
constexpr int AS_WG = 256, AS_B = 4;
template <int HD>
__global__ __launch_bounds__(AS_WG) void k_att_scores(AttSplitArgs a) {
    constexpr int LP = HD / 8, NG = AS_WG / LP;
    __shared__ float redf[AS_WG / 64];
    const int tid = threadIdx.x, h = blockIdx.x, s = blockIdx.y;
    const int kvd = a.kv_heads * HD, kh = h / (a.heads / a.kv_heads);
    const int T = *a.pos + 1;
    const int lo = (int)((int64_t)s * T / ATT_SPLIT), hi = (int)((int64_t)(s + 1) * T / ATT_SPLIT);
    const int grp = tid / LP, c = tid % LP;
    if (s == 0 && tid < HD) a.acc[h * HD + tid] = 0.0;
    // q (raw) and the first batch of keys go out together; q is converted
    // after, so the key loads do not wait for it. Positions past the chunk
    // read a clamped row (position 0 exists for every T) and are masked below.
    const float4 qa = *(const float4*)(a.q + h * HD + 8 * c), qb = *(const float4*)(a.q + h * HD + 8 * c + 4);
    const uint16_t* kb = a.kcache + kh * HD + 8 * c;
    int4 kk[AS_B];
#pragma unroll
    for (int u = 0; u < AS_B; u++) {
        const int t = lo + u * NG + grp, tc = t < hi ? t : (hi > lo ? hi - 1 : 0);
        kk[u] = *(const int4*)(kb + (size_t)tc * kvd);
    }
    const double q8[8] = {(double)qa.x, (double)qa.y, (double)qa.z, (double)qa.w,
                          (double)qb.x, (double)qb.y, (double)qb.z, (double)qb.w};
    float mx = -3.402823466e38f;
    for (int t0 = lo; t0 < hi; t0 += AS_B * NG) {
        if (t0 > lo) {
#pragma unroll
            for (int u = 0; u < AS_B; u++) {
                const int t = t0 + u * NG + grp, tc = t < hi ? t : hi - 1;
                kk[u] = *(const int4*)(kb + (size_t)tc * kvd);
            }
        }
        double d[AS_B];
#pragma unroll
        for (int u = 0; u < AS_B; u++) {
            const uint32_t w[4] = {(uint32_t)kk[u].x, (uint32_t)kk[u].y, (uint32_t)kk[u].z, (uint32_t)kk[u].w};
            double acc = 0.0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc = __builtin_fma(q8[2 * i], (double)uq_half((uint16_t)(w[i] & 0xffff)), acc);
                acc = __builtin_fma(q8[2 * i + 1], (double)uq_half((uint16_t)(w[i] >> 16)), acc);
            }
            d[u] = uq_group_sum<LP>(acc);
        }
#pragma unroll
        for (int u = 0; u < AS_B; u++) {
            const int t = t0 + u * NG + grp;
            if (t < hi) {
                const float sc = (float)d[u] * a.qscale;
                mx = fmaxf(mx, sc);
                if (c == 0) a.scores[(size_t)h * a.max_seq + t] = sc;
            }
        }
    }
    mx = block_max_f<AS_WG>(mx, redf);
    if (tid == 0) a.cmax[h * ATT_SPLIT + s] = mx;
}

// P.V: every chunk workgroup of a head recomputes the global max (from the
// chunk maxima), all exps and their double total (same operations in the
// same order in each workgroup, so the same f32 total); p = e/total for its
// own positions, P.V in double, and the chunk's partial sums are added into
// the accumulator (double atomics: their order only moves the double's last
// bits, far below the one f32 rounding the consumer applies).
template <int HD>
__global__ __launch_bounds__(AS_WG) void k_att_pv(AttSplitArgs a) {
    constexpr int LP = HD / 8, NG = AS_WG / LP, NW = AS_WG / 64;
    extern __shared__ float es[];  // [max_seq]
    __shared__ double red_d[NW];
    __shared__ double part[NW][HD];
    const int tid = threadIdx.x, h = blockIdx.x, s = blockIdx.y;
    const int kvd = a.kv_heads * HD, kh = h / (a.heads / a.kv_heads);
    const int T = *a.pos + 1;
    const int lo = (int)((int64_t)s * T / ATT_SPLIT), hi = (int)((int64_t)(s + 1) * T / ATT_SPLIT);
    const int grp = tid / LP, c = tid % LP;
    // first V batch in flight during the softmax work
    const uint16_t* vb = a.vcache + kh * HD + 8 * c;
    int4 vv[AS_B];
#pragma unroll
    for (int u = 0; u < AS_B; u++) {
        const int t = lo + u * NG + grp;
        vv[u] = t < hi ? *(const int4*)(vb + (size_t)t * kvd) : make_int4(0, 0, 0, 0);
    }
    float mx = -3.402823466e38f;
#pragma unroll
    for (int j = 0; j < ATT_SPLIT; j++) mx = fmaxf(mx, a.cmax[h * ATT_SPLIT + j]);
    const float* sc = a.scores + (size_t)h * a.max_seq;
    double tot = 0.0;  // per thread in position order tid, tid + AS_WG, ...
    for (int t0 = 0; t0 < T; t0 += 4 * AS_WG) {
        float sv[4];  // four scores in flight per thread (index clamped, loads unconditional)
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int t = t0 + u * AS_WG + tid;
            sv[u] = sc[t < T ? t : T - 1];
        }
        float ev[4];  // formed unconditionally, so no load is sunk into the guarded branch
#pragma unroll
        for (int u = 0; u < 4; u++) ev[u] = uq_expf(sv[u] - mx);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int t = t0 + u * AS_WG + tid;
            if (t < T) {
                es[t] = ev[u];
                tot += (double)ev[u];
            }
        }
    }
    tot = block_sum_d<AS_WG>(tot, red_d);  // its barriers also publish es
    const float total = (float)tot;
    double acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = 0.0;
    for (int t0 = lo; t0 < hi; t0 += AS_B * NG) {
        if (t0 > lo) {
#pragma unroll
            for (int u = 0; u < AS_B; u++) {
                const int t = t0 + u * NG + grp;
                vv[u] = t < hi ? *(const int4*)(vb + (size_t)t * kvd) : make_int4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int u = 0; u < AS_B; u++) {
            const int t = t0 + u * NG + grp;
            const float pt = t < hi ? es[t] / total : 0.0f;
            const uint32_t w[4] = {(uint32_t)vv[u].x, (uint32_t)vv[u].y, (uint32_t)vv[u].z, (uint32_t)vv[u].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc[2 * i] = __builtin_fma((double)pt, (double)uq_half((uint16_t)(w[i] & 0xffff)), acc[2 * i]);
                acc[2 * i + 1] = __builtin_fma((double)pt, (double)uq_half((uint16_t)(w[i] >> 16)), acc[2 * i + 1]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = uq_rows_sum<LP>(acc[i]);
    const int wave = tid >> 6, lane = tid & 63;
    if (lane < LP)
#pragma unroll
        for (int i = 0; i < 8; i++) part[wave][8 * lane + i] = acc[i];
    __syncthreads();
    if (tid < HD && hi > lo) {
        double sum = 0.0;
#pragma unroll
        for (int w = 0; w < NW; w++) sum += part[w][tid];
        atomicAdd(&a.acc[h * HD + tid], sum);
    }
}

// ------------------------------------------------------------------ o projection from the accumulator
// Q8_0 matvec whose input is the attention accumulator: the accumulator is
// loaded first, then this workgroup's first row set of weights, then the
// accumulator is rounded to f32 and quantized per 32 into LDS.
template <int LPR, int NBL>
__global__ __launch_bounds__(256) void k_wo_acc(WoArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t lq[MAX_DIM];
    __shared__ float ls[MAX_DIM / 32];
    // K <= min(LPR * NBL * 16, MAX_DIM) (the launcher's checks): PER accumulator values per thread
    constexpr int PK = (LPR * NBL * Q8::UNIT + 255) / 256;
    constexpr int RPW = 64 / LPR, RPB = RPW * 4, PER = PK < MAX_DIM / 256 ? PK : MAX_DIM / 256;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, sub = lane % LPR, grp = lane / LPR;
    const int64_t nu = a.k / Q8::UNIT, K = a.k;
    double av[PER];  // index clamped: all PER loads issue back to back
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = j * 256 + tid;
        av[j] = a.acc[i < K ? i : K - 1];
    }
    const WArgs w{a.w_qs, a.w_d, nullptr};
    const RowSpan sp = row_span<RPB>(a.rows, a.share);
    int64_t row0 = sp.begin;
    Q8::W wv[NBL];
    {
        const int64_t row = row0 + wave * RPW + grp, rr = row < sp.end ? row : sp.end - 1;
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int u = sub + LPR * i, uc = u < nu ? u : (int)nu - 1;
            wv[i] = Q8::load_w(w, rr, nu, uc);
        }
    }
    {
        // uq_quant_lane for the PER blocks of a lane at once: block maxima,
        // then the divisions spread over each 32-lane group (K % 32 == 0, so
        // a block's lanes are all in range or all out of it)
        float v[PER], am[PER], inv[PER], sc[(PER + 31) / 32];
#pragma unroll
        for (int j = 0; j < PER; j++) {
            v[j] = (float)av[j];
            am[j] = uq_group_max<32>(fabsf(v[j]));
        }
        uq_block_recips<PER, 32>(am, inv, sc);
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int i = j * 256 + tid;
            if (i < K) lq[i] = (int8_t)uq_quant_code(v[j], inv[j]);
        }
        // lane r of a 32-lane group holds the scales of its blocks j = r, r + 32, ...
#pragma unroll
        for (int k = 0; k < (PER + 31) / 32; k++) {
            const int j = (tid & 31) + 32 * k, i = j * 256 + (tid & ~31);
            if (j < PER && i < K) ls[i >> 5] = sc[k];
        }
    }
    __syncthreads();
    Q8::X xr[NBL];
    load_xr<Q8, LPR, NBL>(xr, lq, ls, nu, sub);
    for (;;) {
        if (row0 + wave * RPW >= sp.end) break;  // no row of this wave left (wave-uniform)
        const int64_t row = row0 + wave * RPW + grp;
        double acc = 0.0;
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int u = sub + LPR * i;
            const double t = Q8::dot(wv[i], xr[i]);
            acc += u < nu ? t : 0.0;
        }
        acc = uq_group_sum<LPR>(acc);
        if (row < sp.end && sub == 0) a.y[row] = (float)acc;
        row0 += sp.step;
        if (row0 >= sp.end) break;
        const int64_t nrow = row0 + wave * RPW + grp, rr = nrow < sp.end ? nrow : sp.end - 1;
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int u = sub + LPR * i, uc = u < nu ? u : (int)nu - 1;
            wv[i] = Q8::load_w(w, rr, nu, uc);
        }
    }
}

// ------------------------------------------------------------------ decode FFN
// The rows are split evenly over the grid, and in every workgroup the waves
// that hold no rows do the prologue work meanwhile: a wave stalls at issue
// while its CU's weight stream drains, so a wave that also streams weights
// could not start its prologue until then. Down uses one 1024-thread
// workgroup per CU (two 512-thread ones measured slower); gate/up four
// 256-thread workgroups per CU, each with its own prologue wave (1016 ->
// 1041 tok/s against one 1024-thread workgroup; 2 x 512 gave 1027, 8 x 256
// and 8 x 128 were slower).

// Gate/up: 4 rows per wave (16 lanes per row), waves 0..GH_NW-2 hold rows,
// the last wave runs the RMSNorm + quant prologue of the input.
constexpr int GH_RPW = 4, GH_NW = 4, GH_ROWS_MAX = (GH_NW - 1) * GH_RPW;
template <int NBL>
__global__ __launch_bounds__(GH_NW * 64) void k_gateup_h(GateArgs a) {
    constexpr int NC = NBL < MAX_DIM / 256 ? NBL : MAX_DIM / 256;  // dim <= 16 lanes x NBL units x 16
    __shared__ __attribute__((aligned(16))) float lx[NC * 256];
    __shared__ __attribute__((aligned(16))) float lr[NC * 256];
    __shared__ __attribute__((aligned(16))) float lg[NC * 256];
    __shared__ __attribute__((aligned(16))) int8_t sq[NC * 256];
    __shared__ float ssc[NC * 8];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane & 15, grp = lane >> 4;
    const int64_t nu = a.k / Q8::UNIT;
    const RowSpan sp = even_span(a.rows, a.share);
    const int64_t lo = sp.begin, hi = sp.end;
    const bool rows_wave = wave < GH_NW - 1 && wave * GH_RPW < hi - lo;  // wave-uniform
    const int64_t row = lo + wave * GH_RPW + grp, rr = row < hi ? row : hi - 1;
    const WArgs wg{a.g_qs, a.g_d, nullptr}, wu{a.u_qs, a.u_d, nullptr};
    NormQuantWave<NC> nw;
    if (wave == GH_NW - 1) nw.issue(a.nq, lx, lr, lg);
    // The prologue's loads land before this workgroup issues a weight load:
    // a CU holds four of these workgroups, and the last one dispatched would
    // otherwise find its prologue loads queued behind the other three
    // workgroups' weight streams (its prologue ending ~4 us late).
    if (wave == GH_NW - 1) uq_wait_vm0();
    uq_issue_barrier();
    if (wave == GH_NW - 1) nw.finish(a.nq, blockIdx.x == 0, lx, lr, lg, sq, ssc);
    Q8::W gw[NBL], uw[NBL];
    if (rows_wave) {
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int u = sub + 16 * i, uc = u < nu ? u : (int)nu - 1;
            gw[i] = Q8::load_w(wg, rr, nu, uc);
            uw[i] = Q8::load_w(wu, rr, nu, uc);
        }
    }
    __syncthreads();
    if (!rows_wave) return;
    double g = 0.0, uacc = 0.0;
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + 16 * i, uc = u < nu ? u : (int)nu - 1;
        Q8::X x;
        x.a = *(const int4*)(sq + 16 * uc);
        x.s = ssc[uc >> 1];
        const double tg = Q8::dot(gw[i], x), tu = Q8::dot(uw[i], x);
        g += u < nu ? tg : 0.0;
        uacc += u < nu ? tu : 0.0;
    }
    g = uq_group_sum<16>(g);
    uacc = uq_group_sum<16>(uacc);
    if (sub == 0 && row < hi) a.h[row] = uq_silu_mul((float)g, (float)uacc);
}

// Down: one row per wave (64 lanes per row) in waves 0..RW-1, RW = rows per
// workgroup (the same in every workgroup, <= 14); waves RW..15 pull h into
// LDS by DMA and quantize it per 32 (the quant of quant_act, element i =
// 256*c + 4*lane + j, a block = 8 lanes).
constexpr int DH_ROWS_MAX = 14;
template <int NBL>
__global__ __launch_bounds__(1024) void k_down_h(DownArgs a) {
    constexpr int MAXK = NBL * 64 * Q8::UNIT;
    __shared__ __attribute__((aligned(16))) float lh[MAXK];
    __shared__ __attribute__((aligned(16))) int8_t sq[MAXK];
    __shared__ float ssc[MAXK / 32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t nu = a.k / Q8::UNIT, K = a.k;
    const RowSpan sp = even_span(a.rows, a.share);
    const int64_t lo = sp.begin, hi = sp.end;
    const int RW = (int)(a.share + (a.rows > a.share * (int64_t)gridDim.x ? 1 : 0));  // rows of the largest share
    const int64_t row = lo + wave, rr = row < hi ? row : hi - 1;
    const int P = 16 - RW, pw = wave - RW, nch = (int)((K + 255) / 256);
    if (wave >= RW)
        for (int c = pw; c < nch; c += P) {
            const int64_t i = 256 * (int64_t)c + 4 * lane, ic = i < K ? i : K - 4;
            uq_lds_load16(a.h + ic, lh + 256 * c);
        }
    uq_issue_barrier();  // h's loads are queued before any weight load of this CU
    Q8::W wv[NBL];
    if (wave < RW) {
        // no load of these waves is in flight: the wait is free and keeps the
        // compiler's counts exact after the LDS-DMA branch above
        uq_wait_vm0();
        const Q8::R r = Q8::row_ptr(WArgs{a.w_qs, a.w_d, nullptr}, rr, nu);
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int u = lane + 64 * i, uc = u < nu ? u : (int)nu - 1;
            wv[i] = Q8::load_u(r, uc);
        }
        // the scale conversions stay below the last load: here the compiler
        // waits with vmcnt(0) for a single value, which would split the
        // loads into serial batches
        __builtin_amdgcn_sched_barrier(0);
    } else {
        uq_wait_vm0();
        asm volatile("" ::: "memory");
        for (int c = pw; c < nch; c += P) {
            const int64_t i = 256 * (int64_t)c + 4 * lane;
            const float4 v4 = ((const float4*)lh)[64 * c + lane];
            const float v[4] = {v4.x, v4.y, v4.z, v4.w};
            uint32_t packed;
            const float sc = uq_quant4_group8(v, &packed);
            if (i < K) {
                *(uint32_t*)(sq + i) = packed;
                if ((lane & 7) == 0) ssc[i >> 5] = sc;
            }
        }
    }
    __syncthreads();
    if (wave >= RW || row >= hi) return;
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = lane + 64 * i, uc = u < nu ? u : (int)nu - 1;
        Q8::X x;
        x.a = *(const int4*)(sq + 16 * uc);
        x.s = ssc[uc >> 1];
        const double t = Q8::dot(wv[i], x);
        acc += u < nu ? t : 0.0;
    }
    acc = uq_group_sum<64>(acc);
    if (lane == 0) a.y[row] = (float)acc;
}

// ------------------------------------------------------------------ lm_head + argmax partials
template <int LPR, int NBL>
__global__ __launch_bounds__(256) void k_lm_argmax(LmArgs a) {
    constexpr int PK = (LPR * NBL * Q8::UNIT + 255) / 256, NC = PK < MAX_DIM / 256 ? PK : MAX_DIM / 256;
    __shared__ float vs[256];
    __shared__ int ids[256];
    __shared__ unsigned bs[256];
    __shared__ __attribute__((aligned(16))) int8_t lq[NC * 256];
    __shared__ float ls[NC * 8];
    __shared__ double part[4];
    constexpr int RPW = 64 / LPR, RPB = RPW * 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane % LPR, grp = lane / LPR;
    const int64_t nu = a.k / Q8::UNIT;
    float best = -__builtin_inff();
    int id = 0x7fffffff;
    unsigned bad = 0;
    {
        // The output RMSNorm + quant of the input by all four waves (no
        // separate launch): its loads, then the first row set's weights, then
        // its arithmetic while those weights are in flight.
        NormQuantSplit<NC, 4> nw;
        nw.issue(a.nq);
        const WArgs w{a.w_qs, a.w_d, nullptr};
        int64_t row0 = (int64_t)blockIdx.x * RPB;
        Q8::W wv[NBL];
        {
            const int64_t row = row0 + wave * RPW + grp, rr = row < a.rows ? row : a.rows - 1;
            const Q8::R r = Q8::row_ptr(w, rr, nu);
#pragma unroll
            for (int i = 0; i < NBL; i++) {
                const int u = sub + LPR * i, uc = u < nu ? u : (int)nu - 1;
                wv[i] = Q8::load_u(r, uc);
            }
        }
        nw.finish(a.nq, false, part, lq, ls);
        __syncthreads();
        Q8::X xr[NBL];
        load_xr<Q8, LPR, NBL>(xr, lq, ls, nu, sub);
        for (;;) {
            const int64_t row = row0 + wave * RPW + grp;
            double acc = 0.0;
#pragma unroll
            for (int i = 0; i < NBL; i++) {
                const int u = sub + LPR * i;
                const double t = Q8::dot(wv[i], xr[i]);
                acc += u < nu ? t : 0.0;
            }
            const float y = (float)uq_group_sum<LPR>(acc);
            if (row < a.rows && sub == 0) {
                a.logits[row] = y;
                bad |= (__float_as_uint(y) & 0x7f800000u) == 0x7f800000u;
                if (better(y, (int)row, best, id)) {
                    best = y;
                    id = (int)row;
                }
            }
            row0 += (int64_t)gridDim.x * RPB;
            if (row0 >= a.rows) break;
            const int64_t nrow = row0 + wave * RPW + grp, rr = nrow < a.rows ? nrow : a.rows - 1;
            const Q8::R r = Q8::row_ptr(w, rr, nu);
#pragma unroll
            for (int i = 0; i < NBL; i++) {
                const int u = sub + LPR * i, uc = u < nu ? u : (int)nu - 1;
                wv[i] = Q8::load_u(r, uc);
            }
        }
    }
    cand_reduce(best, id, bad, vs, ids, bs);
    if (threadIdx.x == 0) ((Cand*)a.partial)[blockIdx.x] = Cand{best, id, bad, 0u};
}

// Reduces the lm_head partials, publishes the token for the next step,
// appends it to the history and advances the position.
__global__ __launch_bounds__(256) void k_greedy_finish(LmArgs a, int parts) {
    __shared__ float vs[256];
    __shared__ int ids[256];
    __shared__ unsigned bs[256];
    float best = -__builtin_inff();
    int id = 0x7fffffff;
    unsigned bad = 0;
    const Cand* part = (const Cand*)a.partial;
    constexpr int PF = 8;  // partials in flight per thread (index clamped, loads unconditional)
    for (int j0 = threadIdx.x; j0 < parts; j0 += 256 * PF) {
        Cand c[PF];
#pragma unroll
        for (int u = 0; u < PF; u++) {
            const int j = j0 + 256 * u;
            c[u] = part[j < parts ? j : parts - 1];
        }
#pragma unroll
        for (int u = 0; u < PF; u++) {
            if (j0 + 256 * u < parts) {
                bad |= c[u].bad;
                if (better(c[u].v, c[u].id, best, id)) {
                    best = c[u].v;
                    id = c[u].id;
                }
            }
        }
    }
    cand_reduce(best, id, bad, vs, ids, bs);
    if (threadIdx.x == 0) {
        // no candidate (every logit NaN): the flag fails the call, and the id
        // fed to the next step's embedding row must still lie in the vocabulary
        if (id < 0 || (int64_t)id >= a.rows) id = 0;
        a.result[0] = (uint32_t)id;
        a.result[1] = bad;
        a.result[2] |= bad;
        if (a.token) {
            const int pos = *a.pos;
            *a.token = (uint32_t)id;
            if (a.history && pos < a.max_seq) a.history[pos] = (uint32_t)id;
            *a.pos = pos + 1;
        }
    }
}

// ------------------------------------------------------------------ dispatch on units per lane
template <int LPR, template <int, int> class K, class A>
int pick_nbl(int64_t nu, dim3 grid, dim3 block, size_t lds, hipStream_t s, const A& a) {
#define UQ_NB(B)                                                                           \
    if (nu <= (int64_t)LPR * (B)) {                                                        \
        hipLaunchKernelGGL((K<LPR, B>::fn), grid, block, lds, s, a);                      \
        return 0;                                                                          \
    }
    UQ_NB(1) UQ_NB(2) UQ_NB(3) UQ_NB(4) UQ_NB(5) UQ_NB(6) UQ_NB(8) UQ_NB(9) UQ_NB(10) UQ_NB(12) UQ_NB(16)
#undef UQ_NB
    return -1;
}
template <int LPR, int NBL> struct LmArgmax { static constexpr auto fn = k_lm_argmax<LPR, NBL>; };
template <int LPR, int NBL> struct QkvRope { static constexpr auto fn = k_qkv_rope<NBL>; };
template <int LPR, int NBL> struct GateUpH { static constexpr auto fn = k_gateup_h<NBL>; };


int step_lpr(int64_t k) { return k / Q8::UNIT <= 256 ? 32 : 64; }

}  // namespace

int launch_qkv_rope(const QkvArgs& a, hipStream_t s) {
    if (a.dim > MAX_DIM) return -1;
    const int units = (a.heads + 2 * a.kv_heads) * (a.head_dim / 2);
    if (a.dim % 32 || a.nq.dim != a.dim) return -1;
    return pick_nbl<32, QkvRope>(a.dim / Q8::UNIT, dim3((units + 3) / 4), dim3(320), 0, s, a);
}
int launch_attention_split(const AttSplitArgs& a, hipStream_t s) {
    const size_t lds = sizeof(float) * (size_t)a.max_seq;
    if (lds + sizeof(double) * (AS_WG / 64) * (size_t)a.head_dim + 256 > 65536) return -1;
    if (a.heads % a.kv_heads) return -1;
    const dim3 grid((unsigned)a.heads, ATT_SPLIT);
    switch (a.head_dim) {
    case 64:
        hipLaunchKernelGGL(k_att_scores<64>, grid, dim3(AS_WG), 0, s, a);
        hipLaunchKernelGGL(k_att_pv<64>, grid, dim3(AS_WG), lds, s, a);
        return 0;
    case 128:
        hipLaunchKernelGGL(k_att_scores<128>, grid, dim3(AS_WG), 0, s, a);
        hipLaunchKernelGGL(k_att_pv<128>, grid, dim3(AS_WG), lds, s, a);
        return 0;
    case 256:
        hipLaunchKernelGGL(k_att_scores<256>, grid, dim3(AS_WG), 0, s, a);
        hipLaunchKernelGGL(k_att_pv<256>, grid, dim3(AS_WG), lds, s, a);
        return 0;
    default: return -1;
    }
}
template <int LPR, int NBL> struct WoAcc { static constexpr auto fn = k_wo_acc<LPR, NBL>; };
int launch_wo_acc(const WoArgs& a, hipStream_t s) {
    if (a.k > MAX_DIM || a.k % 32) return -1;
    constexpr int RPB = 4 * (64 / 32);
    const int64_t cu = cu_count(), m = (a.rows + cu * RPB - 1) / (cu * RPB);
    int64_t g = m * cu;
    if (g > 2048) g = 2048;
    if (g > a.rows) g = a.rows;
    const unsigned grid = (unsigned)g;
    WoArgs b = a;
    b.share = a.rows / g;
    return pick_nbl<32, WoAcc>(a.k / Q8::UNIT, dim3(grid), dim3(256), 0, s, b);
}
int launch_gateup_h(const GateArgs& a, hipStream_t s) {
    if (a.k > MAX_DIM || a.k % 32 || a.nq.dim != a.k || a.rows <= 0) return -1;
    int64_t g = 4 * cu_count();
    if (g > a.rows) g = a.rows;
    if ((a.rows + g - 1) / g > GH_ROWS_MAX) g = (a.rows + GH_ROWS_MAX - 1) / GH_ROWS_MAX;
    GateArgs b = a;
    b.share = a.rows / g;
    return pick_nbl<16, GateUpH>(a.k / Q8::UNIT, dim3((unsigned)g), dim3(GH_NW * 64), 0, s, b);
}
int launch_down_h(const DownArgs& a, hipStream_t s) {
    if (a.k % 32 || a.k > 9 * 64 * Q8::UNIT || a.rows <= 0) return -1;
    int64_t g = cu_count();
    if (g > a.rows) g = a.rows;
    if ((a.rows + g - 1) / g > DH_ROWS_MAX) g = (a.rows + DH_ROWS_MAX - 1) / DH_ROWS_MAX;
    const int64_t nu = a.k / Q8::UNIT;
    DownArgs b = a;
    b.share = a.rows / g;
    if (nu <= 64 * 3) { hipLaunchKernelGGL(k_down_h<3>, dim3((unsigned)g), dim3(1024), 0, s, b); return 0; }
    if (nu <= 64 * 6) { hipLaunchKernelGGL(k_down_h<6>, dim3((unsigned)g), dim3(1024), 0, s, b); return 0; }
    hipLaunchKernelGGL(k_down_h<9>, dim3((unsigned)g), dim3(1024), 0, s, b);
    return 0;
}
int launch_lm_greedy(const LmArgs& a, hipStream_t s) {
    if (!a.nq.x || !a.nq.gamma || a.nq.dim != a.k || a.k > MAX_DIM || a.k % 32) return -1;
    const int lpr = step_lpr(a.k);
    const int64_t rpb = 4 * (64 / lpr), sets = (a.rows + rpb - 1) / rpb;
    const int parts = (int)(sets < LM_MAX_WG ? sets : LM_MAX_WG);
    const int rc = lpr == 32 ? pick_nbl<32, LmArgmax>(a.k / Q8::UNIT, dim3(parts), dim3(256), 0, s, a)
                             : pick_nbl<64, LmArgmax>(a.k / Q8::UNIT, dim3(parts), dim3(256), 0, s, a);
    if (rc) return rc;
    hipLaunchKernelGGL(k_greedy_finish, dim3(1), dim3(256), 0, s, a, parts);
    return 0;
}

}  // namespace uq
