// Fused decode-step kernels for gfx950.
//
// Per transformer layer:
//   qkv_rope   residual + RMSNorm + quant prologue, q|k|v matvec, q/k bias,
//              RoPE, fp16 K/V store at `pos` (fused_resnorm + quant_act +
//              qkv_dp4a + rope_bias: gpu_fused.cu:193-200, gpu_dp4a.cu:23-59,
//              gpu_ops.cu:235-246)
//   attention  GQA softmax attention over the fp16 cache, output quantized
//              (fused_attention + quant_act, gpu_attention.cu:202-226)
//   o matvec   generic matvec (linear_dp4a)
//   gateup_q   residual + RMSNorm + quant prologue, gate/up matvec, SiLU*up,
//              block-32 quant (gateup_dp4a, gpu_dp4a.cu:60-64)
//   down       generic matvec
// and per token: output RMSNorm, lm_head matvec with per-workgroup argmax,
// greedy finish (greedy_tiles / greedy_finish, gpu_greedy.cu:269-295).
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

namespace uq {
namespace {

constexpr int MAX_DIM = 4096;

// ------------------------------------------------------------------ qkv + rope
// One wave per row pair (32 lanes per row): pair (j, j+hd/2) of a q or k head
// is rotated together; v rows are paired the same way and stored unrotated.
template <int NBL>
__global__ __launch_bounds__(256) void k_qkv_rope(QkvArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t sq[MAX_DIM];
    __shared__ float ssc[MAX_DIM / 32];
    __shared__ double red[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane & 31, grp = lane >> 5;
    const int hd = a.head_dim, half = hd / 2, kvd = a.kv_heads * hd;
    const int nq = a.heads * half, nk = a.kv_heads * half;
    const int pu = blockIdx.x * 4 + wave;
    const bool live = pu < nq + 2 * nk;
    const int region = pu < nq ? 0 : (pu < nq + nk ? 1 : 2);
    const int p = region == 0 ? pu : (region == 1 ? pu - nq : pu - nq - nk);
    const int h = p / half, j = p % half;
    const int ia = h * hd + j, ib = ia + half;  // within the region
    const int rbase = region == 0 ? 0 : (region == 1 ? a.heads * hd : a.heads * hd + kvd);
    const int64_t nu = a.dim / Q8::UNIT;
    const WArgs w{a.w_qs, a.w_d, nullptr};
    NqRegsFor<256, NBL * 32 * Q8::UNIT> nqv;  // dim <= 32 lanes x NBL units x 16
    norm_quant_load<256>(a.nq, nqv);  // activations first: the prologue waits only for them
    Q8::W wv[NBL];
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + 32 * i;
        if (live && u < nu) wv[i] = Q8::load_w(w, rbase + (grp ? ib : ia), nu, u);
    }
    // position-dependent operands of lane 0, fetched before the prologue
    const int pos = *a.pos;
    float cs = 0.0f, sn = 0.0f, ba = 0.0f, bb = 0.0f;
    if (live && lane == 0) {
        const float* bias = region == 0 ? a.bq : (region == 1 ? a.bk : a.bv);
        if (bias) {
            ba = bias[ia];
            bb = bias[ib];
        }
        if (region != 2) {
            cs = a.trig[(size_t)pos * hd + j];
            sn = a.trig[(size_t)pos * hd + half + j];
        }
    }
    norm_quant_finish<256>(a.nq, nqv, blockIdx.x == 0, sq, ssc, red);
    if (!live) return;  // whole wave; no barrier follows
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + 32 * i;
        if (u < nu) {
            Q8::X x;
            x.a = *(const int4*)(sq + 16 * u);
            x.s = ssc[u >> 1];
            acc += Q8::dot(wv[i], x);
        }
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

// ------------------------------------------------------------------ attention
// One 1024-thread workgroup per query head; HD/8 lanes cover one position
// (each lane 8 dims = one 16-byte fp16 load), so a pass covers 1024/(HD/8)
// positions and two passes are issued back to back.
// Scores: q.k in double, butterfly over the position's lanes, * 1/sqrt(hd).
// Softmax: max subtraction, exp, total in double, p = e/total.
// P.V: lane (chunk c, position slice) accumulates 8 dims in double; slices in
// a wave combine by butterfly, the 16 waves through LDS.
constexpr int AT_WG = 1024;
template <int HD>
__global__ __launch_bounds__(AT_WG) void k_attention(AttnArgs a) {
    constexpr int LP = HD / 8, NPASS = AT_WG / LP, NW = AT_WG / 64;
    extern __shared__ double dyn[];  // [NW*HD] P.V partials, then [max_seq] floats
    __shared__ double qd[HD];
    __shared__ double red_d[NW];
    __shared__ float red_f[NW];
    const int tid = threadIdx.x, kvd = a.kv_heads * HD;
    double* part = dyn;
    float* sc = (float*)(dyn + NW * HD);
    const int pos = *a.pos, T = pos + 1;
    const int h = blockIdx.x, kh = h / (a.heads / a.kv_heads);
    if (tid < HD) qd[tid] = (double)a.q[h * HD + tid];
    __syncthreads();
    const int grp = tid / LP, c = tid % LP;
    const uint16_t* kb = a.kcache + kh * HD + 8 * c;
    float mx = -3.402823466e38f;
    for (int t0 = grp; t0 < T; t0 += 2 * NPASS) {
        const int t1 = t0 + NPASS;
        const int4 k0 = *(const int4*)(kb + (size_t)t0 * kvd);
        const int4 k1 = t1 < T ? *(const int4*)(kb + (size_t)t1 * kvd) : make_int4(0, 0, 0, 0);
        const uint32_t w0[4] = {(uint32_t)k0.x, (uint32_t)k0.y, (uint32_t)k0.z, (uint32_t)k0.w};
        const uint32_t w1[4] = {(uint32_t)k1.x, (uint32_t)k1.y, (uint32_t)k1.z, (uint32_t)k1.w};
        double a0 = 0.0, a1 = 0.0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const double q0 = qd[8 * c + 2 * i], q1 = qd[8 * c + 2 * i + 1];
            a0 = __builtin_fma(q0, (double)uq_half((uint16_t)(w0[i] & 0xffff)), a0);
            a0 = __builtin_fma(q1, (double)uq_half((uint16_t)(w0[i] >> 16)), a0);
            a1 = __builtin_fma(q0, (double)uq_half((uint16_t)(w1[i] & 0xffff)), a1);
            a1 = __builtin_fma(q1, (double)uq_half((uint16_t)(w1[i] >> 16)), a1);
        }
        a0 = uq_group_sum<LP>(a0);
        a1 = uq_group_sum<LP>(a1);
        const float s0 = (float)a0 * a.qscale;
        mx = fmaxf(mx, s0);
        if (c == 0) sc[t0] = s0;
        if (t1 < T) {
            const float s1 = (float)a1 * a.qscale;
            mx = fmaxf(mx, s1);
            if (c == 0) sc[t1] = s1;
        }
    }
    mx = block_max_f<AT_WG>(mx, red_f);
    double tot = 0.0;
    for (int t = tid; t < T; t += AT_WG) {
        const float ev = uq_expf(sc[t] - mx);
        sc[t] = ev;
        tot += (double)ev;
    }
    tot = block_sum_d<AT_WG>(tot, red_d);
    const float total = (float)tot;
    for (int t = tid; t < T; t += AT_WG) sc[t] = sc[t] / total;
    __syncthreads();
    double acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = 0.0;
    const uint16_t* vb = a.vcache + kh * HD + 8 * c;
    constexpr int U = 4;
    for (int t0 = grp; t0 < T; t0 += U * NPASS) {
        int4 vv[U];
        double pt[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = t0 + u * NPASS;
            vv[u] = t < T ? *(const int4*)(vb + (size_t)t * kvd) : make_int4(0, 0, 0, 0);
            pt[u] = t < T ? (double)sc[t] : 0.0;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t w[4] = {(uint32_t)vv[u].x, (uint32_t)vv[u].y, (uint32_t)vv[u].z, (uint32_t)vv[u].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc[2 * i] = __builtin_fma(pt[u], (double)uq_half((uint16_t)(w[i] & 0xffff)), acc[2 * i]);
                acc[2 * i + 1] = __builtin_fma(pt[u], (double)uq_half((uint16_t)(w[i] >> 16)), acc[2 * i + 1]);
            }
        }
    }
    // lanes with the same chunk in a wave: c = lane % LP
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = uq_rows_sum<LP>(acc[i]);
    const int wave = tid >> 6, lane = tid & 63;
    if (lane < LP)
#pragma unroll
        for (int i = 0; i < 8; i++) part[wave * HD + 8 * lane + i] = acc[i];
    __syncthreads();
    if (tid < HD) {
        double s = 0.0;
        for (int w = 0; w < NW; w++) s += part[w * HD + tid];
        const float o = (float)s;
        if (a.out) a.out[h * HD + tid] = o;
        float qs;
        const int8_t qv = uq_quant_lane(o, &qs);
        a.xq[h * HD + tid] = qv;
        if ((tid & 31) == 0) a.xs[(h * HD + tid) >> 5] = qs;
    }
}

// ------------------------------------------------------------------ gate/up + SiLU + quant
// 32 consecutive rows per 1024-thread workgroup (two rows per wave), so the
// block-32 quantization of the outputs stays inside the workgroup.
template <int NBL>
__global__ __launch_bounds__(1024) void k_gateup_q(GateArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t sq[MAX_DIM];
    __shared__ float ssc[MAX_DIM / 32];
    __shared__ double red[16];
    __shared__ float ys[32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane & 31, grp = lane >> 5;
    const int64_t nu = a.k / Q8::UNIT;
    const int64_t row = (int64_t)blockIdx.x * 32 + wave * 2 + grp;
    const WArgs wg{a.g_qs, a.g_d, nullptr}, wu{a.u_qs, a.u_d, nullptr};
    NqRegsFor<1024, NBL * 32 * Q8::UNIT> nqv;  // dim <= 32 lanes x NBL units x 16
    norm_quant_load<1024>(a.nq, nqv);  // activations first: the prologue waits only for them
    Q8::W gw[NBL], uw[NBL];
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + 32 * i;
        if (u < nu) {
            gw[i] = Q8::load_w(wg, row, nu, u);
            uw[i] = Q8::load_w(wu, row, nu, u);
        }
    }
    norm_quant_finish<1024>(a.nq, nqv, blockIdx.x == 0, sq, ssc, red);
    double g = 0.0, uacc = 0.0;
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int u = sub + 32 * i;
        if (u < nu) {
            Q8::X x;
            x.a = *(const int4*)(sq + 16 * u);
            x.s = ssc[u >> 1];
            g += Q8::dot(gw[i], x);
            uacc += Q8::dot(uw[i], x);
        }
    }
    g = uq_group_sum<32>(g);
    uacc = uq_group_sum<32>(uacc);
    if (sub == 0) ys[wave * 2 + grp] = uq_silu_mul((float)g, (float)uacc);
    __syncthreads();
    if (threadIdx.x < 32) {
        const float v = ys[threadIdx.x];
        const int64_t r = (int64_t)blockIdx.x * 32 + threadIdx.x;
        if (a.out) a.out[r] = v;
        float s;
        const int8_t q = uq_quant_lane(v, &s);
        a.oq[r] = q;
        if (threadIdx.x == 0) a.os[blockIdx.x] = s;
    }
}

// ------------------------------------------------------------------ lm_head + argmax partials
template <int LPR, int NBL>
__global__ __launch_bounds__(256) void k_lm_argmax(LmArgs a) {
    __shared__ float vs[256];
    __shared__ int ids[256];
    __shared__ unsigned bs[256];
    constexpr int RPW = 64 / LPR, RPB = RPW * 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane % LPR, grp = lane / LPR;
    const int64_t nu = a.k / Q8::UNIT;
    float best = -__builtin_inff();
    int id = 0x7fffffff;
    unsigned bad = 0;
    {
        Q8::X xr[NBL];
        load_xr<Q8, LPR, NBL>(xr, a.xq, a.xs, nu, sub);
        const WArgs w{a.w_qs, a.w_d, nullptr};
        for (int64_t row0 = (int64_t)blockIdx.x * RPB; row0 < a.rows; row0 += (int64_t)gridDim.x * RPB) {
            const int64_t row = row0 + wave * RPW + grp;
            if (row < a.rows) {
                const float y = (float)row_dot<Q8, LPR, NBL>(w, row, nu, sub, xr);
                if (sub == 0) {
                    a.logits[row] = y;
                    bad |= (__float_as_uint(y) & 0x7f800000u) == 0x7f800000u;
                    if (better(y, (int)row, best, id)) {
                        best = y;
                        id = (int)row;
                    }
                }
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
    for (int j = threadIdx.x; j < parts; j += 256) {
        const Cand c = part[j];
        bad |= c.bad;
        if (better(c.v, c.id, best, id)) {
            best = c.v;
            id = c.id;
        }
    }
    cand_reduce(best, id, bad, vs, ids, bs);
    if (threadIdx.x == 0) {
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
template <int LPR, int NBL> struct GateUpQ { static constexpr auto fn = k_gateup_q<NBL>; };

int step_lpr(int64_t k) { return k / Q8::UNIT <= 256 ? 32 : 64; }

}  // namespace

int launch_qkv_rope(const QkvArgs& a, hipStream_t s) {
    if (a.dim > MAX_DIM) return -1;
    const int units = (a.heads + 2 * a.kv_heads) * (a.head_dim / 2);
    return pick_nbl<32, QkvRope>(a.dim / Q8::UNIT, dim3((units + 3) / 4), dim3(256), 0, s, a);
}
int launch_attention_q(const AttnArgs& a, hipStream_t s) {
    const size_t lds = sizeof(double) * (size_t)(AT_WG / 64) * a.head_dim + sizeof(float) * (size_t)a.max_seq;
    if (lds + sizeof(double) * a.head_dim + 256 > 65536) return -1;
    switch (a.head_dim) {
    case 64: hipLaunchKernelGGL(k_attention<64>, dim3(a.heads), dim3(AT_WG), lds, s, a); return 0;
    case 128: hipLaunchKernelGGL(k_attention<128>, dim3(a.heads), dim3(AT_WG), lds, s, a); return 0;
    case 256: hipLaunchKernelGGL(k_attention<256>, dim3(a.heads), dim3(AT_WG), lds, s, a); return 0;
    default: return -1;
    }
}
int launch_gateup_q(const GateArgs& a, hipStream_t s) {
    if (a.k > MAX_DIM || a.rows % 32) return -1;
    return pick_nbl<32, GateUpQ>(a.k / Q8::UNIT, dim3((unsigned)(a.rows / 32)), dim3(1024), 0, s, a);
}
int launch_lm_greedy(const LmArgs& a, hipStream_t s) {
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
