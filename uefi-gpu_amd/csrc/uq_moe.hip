// MoE expert FFN for one token on gfx950: softmax routing with stable top-k,
// the selected experts' gate/up matvecs with SiLU*up and block-32 quant, their
// down matvecs and the rank-ordered weighted combine, plus the shared expert.
//
// Replaces Forward::ffn (driver/src/frontier_forward.rs:164-199) and its
// descriptor-driven multi-matvec launch (frontier_multi_matvec,
// driver/kernels/frontier_quant.cu:71-93; pack, frontier_dispatch.rs:12-31).
// The reference moves experts between SSD, CPU and a 12 GB card; here every
// expert sits in an HBM-resident bank (experts stacked by rows in one repacked
// weight per projection), and the routing result stays on the device: the
// gate/up and down kernels turn the selected expert ids into row offsets of
// the bank, the role the 48-byte job table plays in the reference.
//
// Arithmetic (same as the oracle): softmax with max subtraction and a f32
// running sum in expert order, stable selection (score descending, id
// ascending), weights p/sum(top-k) with the f32 sum in rank order; int8
// activations per 32; exact double sums per row; SiLU as g * (1/(1+exp(-g)));
// out = sum over ranks of (w * v) as separate multiply then add, then the
// shared expert with sigmoid(shexp_gate . x).
#include "uq_device.h"
#include "uq_units.h"
#include "uq_blockops.h"
#include "uq_internal.h"
#include "../../include/uq.h"

#include <cmath>
#include <cstring>
#include <string>
#include <vector>

namespace uq {
namespace {

constexpr int MAX_EXPERTS = 1024, MAX_TOPK = 16, MAX_D = 8192, MAX_F = 4096;

struct MoeDev {
    const float* x;          // [D] input
    const float* logits;     // [E] router logits
    const float* sh_gate;    // [D] f32 shared-expert gate vector (may be null: weight 1)
    int8_t* xq;              // [D]
    float* xs;               // [D/32]
    int32_t* ids;            // [top_k]
    float* wts;              // [top_k + 1]: routed weights, then the shared weight
    unsigned* status;        // [0] != 0: non-finite input / router failure
    int8_t* midq;            // [(top_k+1)][F]
    float* mids;             // [(top_k+1)][F/32]
    float* out;              // [D]
    int D, F, E, top_k;
};

// ------------------------------------------------------------------ routing + gate/up
// One launch does routing, input quant and the gate/up projections. Every
// 512-thread workgroup owns 32 consecutive rows of one expert slot's gate and
// up matrices (16 lanes per row); slot < top_k is the routed expert of that
// rank, slot == top_k the shared expert. Each workgroup recomputes the routing
// (128 scores from 512 bytes of logits: cheaper than a dependent launch) and
// quantizes x into LDS; workgroup (0, 0) publishes ids, weights and the
// status flag, workgroup (top_k, 0) the shared expert's sigmoid gate. The
// shared slot's weight loads are issued before the routing work.
constexpr int GU_WG = 512;

struct RouteLds {
    float p[MAX_EXPERTS];
    unsigned long long key[GU_WG / 4];  // rank keys of up to 128 experts
    int part[GU_WG];         // partial ranks of the 2nd..RQ-th thread of an expert
    int sid[MAX_TOPK];
    double red[GU_WG / 64];
    float redf[GU_WG / 64];
    float sum;
    unsigned badw[GU_WG / 64];  // per wave: any non-finite input seen
};

// Routing arithmetic (the oracle's, frontier_forward.rs:47-51): softmax with
// max subtraction and an f32 running sum in expert order; stable top-k (score
// descending, id ascending).

// Routing by the whole workgroup. Up to 128 experts, wave 0 alone forms the
// max, exps, the f32 running sum in expert order and p = e / sum (two experts
// per lane, no workgroup barrier) while waves 1.. run `side` (the input
// quant); then stable ranks by four threads per expert against LDS broadcast
// reads of a -1-padded table. More experts: GU_PE per thread with a barrier
// between phases (max by DPP per wave then across waves, exps to LDS, the
// running sum by lane 0 of wave 0 while waves 1.. run `side`, p in place,
// ranks by two or one threads per expert). Leaves p in L.p and the top-k ids
// in L.sid, published by the barrier it ends on, and the OR of every
// thread's non-finite flag in `bad`.
constexpr int GU_PE = (MAX_EXPERTS + GU_WG - 1) / GU_WG;
template <class Side>
__device__ float route_par(const MoeDev& a, const float* lg, float lg_hi, RouteLds& L, unsigned& bad, Side side) {
    const int t = threadIdx.x, E = a.E;
    // each wave's flag, written by its lane 0 before a barrier (no clearing
    // step that could race with another wave's write)
    auto publish_bad = [&]() {
        const unsigned any = __any(bad != 0u) ? 1u : 0u;
        if ((t & 63) == 0) L.badw[t >> 6] = any;
    };
    auto gather_bad = [&]() {
        unsigned b = 0u;
#pragma unroll
        for (int w = 0; w < GU_WG / 64; w++) b |= L.badw[w];
        bad = b;
    };
    if (((E + 3) & ~3) <= GU_WG / 4) {
        // Up to 128 experts: wave 0 alone forms the max (wave reduction), the
        // exps, the running sum and p for experts t and t + 64 of each lane --
        // no workgroup barrier -- while waves 1.. run `side`. The operations
        // and their order are those of the general path below.
        if (t < 64) {
            const bool in0 = t < E, in1 = t + 64 < E;
            bad |= (in0 && !isfinite(lg[0])) | (in1 && !isfinite(lg_hi));
            float m = -__builtin_inff();
            if (in0) m = fmaxf(m, lg[0]);
            if (in1) m = fmaxf(m, lg_hi);
            const float mx = uq_group_max<64>(m);
            // entries past E hold -1 up to 128 entries (the rank table)
            const float e0 = in0 ? uq_expf(lg[0] - mx) : -1.0f, e1 = in1 ? uq_expf(lg_hi - mx) : -1.0f;
            L.p[t] = e0;
            L.p[t + 64] = e1;
            if (t < a.top_k) L.sid[t] = t;
            // this wave's LDS writes are seen by its own later reads in order
            asm volatile("" ::: "memory");
            __builtin_amdgcn_wave_barrier();
            float sl = 0.0f;
            if (t == 0) {
                const float4* p4 = (const float4*)L.p;
                int q = 0;
                for (; q + 8 <= E / 4; q += 8) {
                    float4 v[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) v[u] = p4[q + u];
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        sl = sl + v[u].x;
                        sl = sl + v[u].y;
                        sl = sl + v[u].z;
                        sl = sl + v[u].w;
                    }
                }
                for (; q < E / 4; q++) {
                    const float4 v = p4[q];
                    sl = sl + v.x;
                    sl = sl + v.y;
                    sl = sl + v.z;
                    sl = sl + v.w;
                }
                for (int e = E & ~3; e < E; e++) sl = sl + L.p[e];
                L.sum = sl;
            }
            const float sum = __shfl(sl, 0, 64);
            const float p0 = e0 / sum, p1 = e1 / sum;
            if (in0) L.p[t] = p0;
            if (in1) L.p[t + 64] = p1;
            // rank key: p's bits (p >= +0, so they order as p does) above
            // 127 - e (a tie goes to the lower id); 0 for a slot past E, which
            // is never above a real key. Unique keys, so the top-k is one
            // permutation even if p holds a NaN (the status flag reports it).
            L.key[t] = in0 ? ((unsigned long long)__float_as_uint(p0) << 7) | (unsigned)(127 - t) : 0ull;
            L.key[t + 64] = in1 ? ((unsigned long long)__float_as_uint(p1) << 7) | (unsigned)(63 - t) : 0ull;
        } else {
            side();
        }
        publish_bad();
        __syncthreads();
        // stable ranks on the keys: four threads per expert, each counting
        // the keys above its expert's among a quarter of the table (the same
        // order as p descending, id ascending)
        constexpr int NE = GU_WG / 4;
        const int e = t % NE, q = t / NE;
        const unsigned long long kv = L.key[e];
        int rank = 0;
#pragma unroll
        for (int u = 0; u < NE / 4; u++) rank += L.key[q * (NE / 4) + u] > kv ? 1 : 0;
        if (q > 0) L.part[(q - 1) * NE + e] = rank;
        __syncthreads();
        if (q == 0 && e < E) {
#pragma unroll
            for (int k = 1; k < 4; k++) rank += L.part[(k - 1) * NE + e];
            if (rank < a.top_k) L.sid[rank] = e;
        }
        __syncthreads();
        gather_bad();
        return L.sum;
    }
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < GU_PE; j++) {
        const int e = j * GU_WG + t;
        if (e < E) {
            bad |= !isfinite(lg[j]);
            mx = fmaxf(mx, lg[j]);
        }
    }
    mx = block_max_f<GU_WG>(mx, L.redf);
#pragma unroll
    for (int j = 0; j < GU_PE; j++) {
        const int e = j * GU_WG + t;
        if (e < E) L.p[e] = uq_expf(lg[j] - mx);
    }
    // entries past E hold -1: never above a score, never equal to one
    const int E4 = (E + 3) & ~3;
    if (t < E4 - E) L.p[E + t] = -1.0f;
    // with a NaN score no rank is unique; the slots then keep ids 0..k-1 and
    // the status flag reports the input
    if (t < a.top_k) L.sid[t] = t;
    __syncthreads();
    if (t < 64) {
        if (t == 0) {
        const float4* p4 = (const float4*)L.p;
        float s = 0.0f;
        int q = 0;
        for (; q + 8 <= E / 4; q += 8) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = p4[q + u];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                s = s + v[u].x;
                s = s + v[u].y;
                s = s + v[u].z;
                s = s + v[u].w;
            }
        }
        for (; q < E / 4; q++) {
            const float4 v = p4[q];
            s = s + v.x;
            s = s + v.y;
            s = s + v.z;
            s = s + v.w;
        }
        for (int e = E & ~3; e < E; e++) s = s + L.p[e];
        L.sum = s;
        }
    } else {
        side();
    }
    __syncthreads();
    const float sum = L.sum;
    float pe[GU_PE];
#pragma unroll
    for (int j = 0; j < GU_PE; j++) {
        const int e = j * GU_WG + t;
        pe[j] = e < E ? L.p[e] / sum : 0.0f;
        if (e < E) L.p[e] = pe[j];  // each thread rewrites only its own entries
    }
    // every flag (logits in the max pass, the input in `side`) is final here
    publish_bad();
    __syncthreads();
    // stable ranks: RQ threads per expert (2 up to 256 experts, else 1), each
    // comparing against every RQ-th float4 of the probabilities with all of
    // its LDS reads issued before the compares; partial counts meet in LDS
    const float4* p4 = (const float4*)L.p;
    const int RQ = E4 <= GU_WG / 2 ? 2 : 1;
    for (int e0 = 0; e0 < E4; e0 += GU_WG / RQ) {
        const int e = e0 + t % (GU_WG / RQ), q = t / (GU_WG / RQ);
        const float v = e < E ? L.p[e] : 0.0f;
        int rank = 0;
        constexpr int CH = 8;  // float4 reads in flight
        for (int c0 = q; c0 < E4 / 4; c0 += RQ * CH) {
            float4 w[CH];
#pragma unroll
            for (int u = 0; u < CH; u++) {
                const int c = c0 + RQ * u;
                w[u] = c < E4 / 4 ? p4[c] : make_float4(-1.0f, -1.0f, -1.0f, -1.0f);
            }
#pragma unroll
            for (int u = 0; u < CH; u++) {
                // bitwise (not short-circuit) tests keep the loop branch-free;
                // the -1 padding is never above a probability nor equal to one
                const int i0 = 4 * (c0 + RQ * u);
                rank += (int)(w[u].x > v) | ((int)(w[u].x == v) & (int)(i0 < e));
                rank += (int)(w[u].y > v) | ((int)(w[u].y == v) & (int)(i0 + 1 < e));
                rank += (int)(w[u].z > v) | ((int)(w[u].z == v) & (int)(i0 + 2 < e));
                rank += (int)(w[u].w > v) | ((int)(w[u].w == v) & (int)(i0 + 3 < e));
            }
        }
        if (RQ > 1) {
            const int el = e % (GU_WG / RQ);
            if (q > 0 && e < E) L.part[(q - 1) * (GU_WG / RQ) + el] = rank;
            __syncthreads();
            if (q == 0 && e < E) {
                for (int k = 1; k < RQ; k++) rank += L.part[(k - 1) * (GU_WG / RQ) + el];
                if (rank < a.top_k) L.sid[rank] = e;
            }
            __syncthreads();
        } else if (e < E && rank < a.top_k) {
            L.sid[rank] = e;
        }
    }
    __syncthreads();
    gather_bad();
    return sum;
}

// this lane's gate/up units of row `row`: loads, then dots (16 lanes per row)
template <class KQ, int NBL>
struct GuLane {
    typename KQ::W gw[NBL], uw[NBL];
    __device__ void load(WArgs wg, WArgs wu, int64_t row, int64_t nu, int sub) {
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int un = sub + 16 * i, uc = un < nu ? un : (int)nu - 1;
            gw[i] = KQ::load_w(wg, row, nu, uc);
            uw[i] = KQ::load_w(wu, row, nu, uc);
        }
    }
    __device__ float silu_mul(const int8_t* xq, const float* xs, int64_t nu, int sub) const {
        typename KQ::X xr[NBL];
        load_xr<KQ, 16, NBL>(xr, xq, xs, nu, sub);
        double g = 0.0, u = 0.0;
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int un = sub + 16 * i, uc = un < nu ? un : (int)nu - 1;
            const double tg = KQ::dot(gw[i], xr[i], uc), tu = KQ::dot(uw[i], xr[i], uc);
            g += un < nu ? tg : 0.0;
            u += un < nu ? tu : 0.0;
        }
        g = uq_group_sum<16>(g);
        u = uq_group_sum<16>(u);
        const float gf = (float)g, uf = (float)u;
        const float sg = gf * uq_sigmoid(gf);
        return sg * uf;
    }
};

template <class KR, int NR, class KS, int NS>
__global__ __launch_bounds__(GU_WG) void k_moe_gateup(MoeDev a, WArgs rg, WArgs ru, WArgs sg, WArgs su) {
    __shared__ RouteLds L;
    __shared__ __attribute__((aligned(16))) int8_t lxq[MAX_D];
    __shared__ float lxs[MAX_D / 32];
    __shared__ float ys[32];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, sub = lane & 15, grp = lane >> 4;
    // the shared expert's row blocks (the heaviest: Q8_0 rows) take the first
    // block indices so that they are dispatched first; routed slots follow
    const int blocks = a.F / 32;
    const int bi = (int)blockIdx.x < blocks ? (int)blockIdx.x + a.top_k * blocks : (int)blockIdx.x - blocks;
    const int slot = bi / blocks, rb = bi % blocks;
    const bool shared = slot == a.top_k;
    const int D = a.D;
    // logits and x up front; waves 1..7 quantize x (4 values per lane, a
    // 32-block = 8 lanes) while wave 0 forms the softmax sum
    float lg[GU_PE];
#pragma unroll
    for (int j = 0; j < GU_PE; j++) {
        const int e = j * GU_WG + t;
        lg[j] = e < a.E ? a.logits[e] : 0.0f;
    }
    const float lg_hi = a.logits[t + 64 < a.E ? t + 64 : a.E - 1];  // wave 0's second expert (up to 128)
    constexpr int QT = GU_WG - 64, QP = (MAX_D + 4 * QT - 1) / (4 * QT);
    const int qt = t - 64;
    float4 xv[QP];
#pragma unroll
    for (int j = 0; j < QP; j++) {
        const int i = (j * QT + qt) * 4;
        xv[j] = (qt >= 0 && i < D) ? *(const float4*)(a.x + i) : float4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    GuLane<KS, NS> sl;
    const int64_t srow = (int64_t)rb * 32 + wave * 4 + grp;
    if (shared) sl.load(sg, su, srow, D / KS::UNIT, sub);
    unsigned bad = 0;
    // i < D is uniform over each 8-lane block group (D is a multiple of 32)
    auto quant_x = [&]() {
#pragma unroll
        for (int j = 0; j < QP; j++) {
            const int i = (j * QT + qt) * 4;
            if (i < D) {
                const float v[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
                bad |= !isfinite(v[0]) | !isfinite(v[1]) | !isfinite(v[2]) | !isfinite(v[3]);
                uint32_t pk;
                const float sc = uq_quant4_group8(v, &pk);
                *(uint32_t*)(lxq + i) = pk;
                if ((qt & 7) == 0) lxs[i >> 5] = sc;
            }
        }
    };
    // route_par ends on a barrier that publishes L.p / L.sid and lxq / lxs,
    // and leaves in `bad` the OR of every thread's non-finite flag. The
    // shared expert's workgroups need no routing, only the quantized input:
    // their own weight loads, issued first, would hold up their logits load
    // and make them the launch's last workgroups (routing done at 4.6 us
    // against 2.9 in the routed ones, in a stamped build).
    float sum = 0.0f;
    if (!shared) {
        sum = route_par(a, lg, lg_hi, L, bad, quant_x);
    } else {
        if (t >= 64) quant_x();  // waves 1.. (quant_x's element index is t - 64)
        __syncthreads();
    }
    float v;
    if (!shared) {
        // routed expert: its weight loads go out before anything else waits
        const int e = L.sid[slot];
        const int ec = e < 0 ? 0 : (e >= a.E ? a.E - 1 : e);
        GuLane<KR, NR> rl;
        rl.load(rg, ru, (int64_t)ec * a.F + srow, D / KR::UNIT, sub);
        if (bi == 0 && t == 0) {
            float tot = 0.0f;
            for (int k = 0; k < a.top_k; k++) tot = tot + L.p[L.sid[k]];
            if (!(sum > 0.0f) || !isfinite(sum) || !(tot > 0.0f)) bad = 1;
            for (int k = 0; k < a.top_k; k++) {
                a.ids[k] = L.sid[k];
                a.wts[k] = L.p[L.sid[k]] / tot;
            }
            a.status[0] = bad;
        }
        v = rl.silu_mul(lxq, lxs, D / KR::UNIT, sub);
    } else {
        if (rb == 0) {
            // shared expert weight sigmoid(shexp_gate . x), dot in double
            double dot = 0.0;
            if (a.sh_gate)
                for (int i = t; i < D; i += GU_WG) dot = __builtin_fma((double)a.sh_gate[i], (double)a.x[i], dot);
            dot = block_sum_d<GU_WG>(dot, L.red);
            if (t == 0) a.wts[a.top_k] = a.sh_gate ? uq_sigmoid((float)dot) : 1.0f;
        }
        v = sl.silu_mul(lxq, lxs, D / KS::UNIT, sub);
    }
    if (sub == 0) ys[wave * 4 + grp] = v;
    __syncthreads();
    if (t < 32) {
        const float y = ys[t];
        float s;
        const int8_t q = uq_quant_lane(y, &s);
        a.midq[(size_t)slot * a.F + rb * 32 + t] = q;
        if (t == 0) a.mids[(size_t)slot * (a.F / 32) + rb] = s;
    }
}

// Routed expert id of slot k, clamped into the bank: a row address is never
// formed from an id outside [0, E).
__device__ __forceinline__ int expert_id(const MoeDev& a, int k) {
    const int e = a.ids[k];
    return e < 0 ? 0 : (e >= a.E ? a.E - 1 : e);
}

// ------------------------------------------------------------------ down + combine
// Two output rows per 256-thread workgroup. Waves 0 and 1 take the routed
// experts of rows r and r+1: lane group g of LS lanes is slot k = pass*SPW + g
// and its lanes cover that expert's down row (NR units each); waves 2 and 3
// take the shared expert's row over all 64 lanes (NS units each). Every load
// of a pass is issued before its dots. The per-slot sums meet in LDS and one
// lane per row combines them in rank order as out = out + w*v (separate
// multiply and add), shared expert last.
template <class KR, int LS, int NR, class KS, int NS>
__global__ __launch_bounds__(256) void k_moe_down(MoeDev a, WArgs rd, WArgs sd) {
    constexpr int SPW = 64 / LS;
    __shared__ float vs[2][MAX_TOPK + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = wave & 1;
    const int64_t row = (int64_t)blockIdx.x * 2 + half;
    const bool live = row < a.D;
    const int64_t rr = live ? row : a.D - 1;
    if (wave < 2) {
        const int64_t nu = a.F / KR::UNIT;
        const int g = lane / LS, sub = lane % LS;
        for (int k0 = 0; k0 < a.top_k; k0 += SPW) {
            const int k = k0 + g, kc = k < a.top_k ? k : a.top_k - 1;
            const int64_t r = (int64_t)expert_id(a, kc) * a.D + rr;
            const int8_t* xq = a.midq + (size_t)kc * a.F;
            const float* xs = a.mids + (size_t)kc * (a.F / 32);
            typename KR::W wv[NR];
#pragma unroll
            for (int i = 0; i < NR; i++) {
                const int u = sub + LS * i, uc = u < nu ? u : (int)nu - 1;
                wv[i] = KR::load_w(rd, r, nu, uc);
            }
            typename KR::X xr[NR];
            load_xr<KR, LS, NR>(xr, xq, xs, nu, sub);
            double acc = 0.0;
#pragma unroll
            for (int i = 0; i < NR; i++) {
                const int u = sub + LS * i, uc = u < nu ? u : (int)nu - 1;
                const double t = KR::dot(wv[i], xr[i], uc);
                acc += u < nu ? t : 0.0;
            }
            acc = uq_group_sum<LS>(acc);
            if (sub == 0 && k < a.top_k) vs[half][k] = (float)acc;
        }
    } else {
        const int64_t nu = a.F / KS::UNIT;
        const int8_t* xq = a.midq + (size_t)a.top_k * a.F;
        const float* xs = a.mids + (size_t)a.top_k * (a.F / 32);
        typename KS::W wv[NS];
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const int u = lane + 64 * i, uc = u < nu ? u : (int)nu - 1;
            wv[i] = KS::load_w(sd, rr, nu, uc);
        }
        typename KS::X xr[NS];
        load_xr<KS, 64, NS>(xr, xq, xs, nu, lane);
        double acc = 0.0;
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const int u = lane + 64 * i, uc = u < nu ? u : (int)nu - 1;
            const double t = KS::dot(wv[i], xr[i], uc);
            acc += u < nu ? t : 0.0;
        }
        acc = uq_group_sum<64>(acc);
        if (lane == 0) vs[half][a.top_k] = (float)acc;
    }
    __syncthreads();
    if (threadIdx.x < 2 && (int64_t)blockIdx.x * 2 + threadIdx.x < a.D) {
        float o = 0.0f;
        for (int k = 0; k <= a.top_k; k++) {
            const float tv = a.wts[k] * vs[threadIdx.x][k];
            o = o + tv;
        }
        a.out[(int64_t)blockIdx.x * 2 + threadIdx.x] = o;
    }
}

}  // namespace
}  // namespace uq

using namespace uq;

struct uq_moe {
    int32_t D = 0, F = 0, E = 0, K = 0;
    uint32_t kind = 0, shared_kind = 0;
    Weight gate, up, down;      // expert banks: rows stacked expert-major
    Weight sgate, sup, sdown;   // shared expert
    std::vector<uint8_t> hg, hu, hd;  // host staging of the banks until finalize
    std::vector<char> have;
    bool ready = false, shared_set = false;
    float* sh_vec = nullptr;
    // device state
    float *x = nullptr, *logits = nullptr, *out = nullptr, *xs = nullptr, *wts = nullptr, *mids = nullptr;
    int8_t *xq = nullptr, *midq = nullptr;
    int32_t* ids = nullptr;
    unsigned* status = nullptr;
    std::vector<void*> owned;
};

static void free_weight(Weight& w) {
    if (w.alloc) hipFree(w.alloc);
    w = Weight{};
}

static int upload_into(Weight& dst, uint32_t kind, int64_t n, int64_t m, const void* data, size_t bytes) {
    return upload_weight(kind, n, m, data, bytes, dst, /*bank=*/true);
}

extern "C" {

int uq_moe_create(int32_t dim, int32_t ff, int32_t experts, int32_t top_k, uint32_t expert_kind, uq_moe_t* out) {
    if (!out) return set_error(ERR_ARG, "moe_create: null pointer");
    if (!uq_stream()) return set_error(ERR_ARG, "uq_init has not been called");
    if (dim <= 0 || dim > MAX_D || dim % 256 || ff <= 0 || ff > MAX_F || ff % 256 || experts <= 0 ||
        experts > MAX_EXPERTS || top_k <= 0 || top_k > MAX_TOPK || top_k > experts)
        return set_error(ERR_SHAPE, "moe_create: unsupported shape");
    if (expert_kind != KIND_Q3_K && expert_kind != KIND_Q4_K && expert_kind != KIND_Q8_0)
        return set_error(ERR_QUANT_TYPE, "moe_create: experts must be Q3_K, Q4_K or Q8_0");
    uq_moe* m = new uq_moe();
    m->D = dim;
    m->F = ff;
    m->E = experts;
    m->K = top_k;
    m->kind = expert_kind;
    const int64_t rbg = row_bytes(expert_kind, dim), rbd = row_bytes(expert_kind, ff);
    m->hg.resize((size_t)(rbg * ff * experts));
    m->hu.resize((size_t)(rbg * ff * experts));
    m->hd.resize((size_t)(rbd * dim * experts));
    m->have.assign((size_t)experts, 0);
    *out = m;
    return OK;
}

int uq_moe_info(uq_moe_t m, int32_t* dim, int32_t* ff, int32_t* experts, int32_t* top_k, uint32_t* expert_kind) {
    if (!m) return set_error(ERR_ARG, "moe_info: null handle");
    if (dim) *dim = m->D;
    if (ff) *ff = m->F;
    if (experts) *experts = m->E;
    if (top_k) *top_k = m->K;
    if (expert_kind) *expert_kind = m->kind;
    return OK;
}

int uq_moe_free(uq_moe_t m) {
    if (!m) return OK;
    hipStreamSynchronize((hipStream_t)uq_stream());
    for (Weight* w : {&m->gate, &m->up, &m->down, &m->sgate, &m->sup, &m->sdown}) free_weight(*w);
    for (void* p : m->owned) hipFree(p);
    delete m;
    return OK;
}

int uq_moe_set_expert(uq_moe_t m, int32_t e, const void* gate, const void* up, const void* down) {
    if (!m || !gate || !up || !down) return set_error(ERR_ARG, "moe_set_expert: null pointer");
    if (m->ready) return set_error(ERR_ARG, "moe_set_expert: layer already finalized");
    if (e < 0 || e >= m->E) return set_error(ERR_SHAPE, "moe_set_expert: expert id out of range");
    const size_t bg = (size_t)(row_bytes(m->kind, m->D) * m->F), bd = (size_t)(row_bytes(m->kind, m->F) * m->D);
    std::memcpy(m->hg.data() + bg * e, gate, bg);
    std::memcpy(m->hu.data() + bg * e, up, bg);
    std::memcpy(m->hd.data() + bd * e, down, bd);
    m->have[(size_t)e] = 1;
    return OK;
}

int uq_moe_set_shared(uq_moe_t m, uint32_t kind, const void* gate, const void* up, const void* down,
                      const float* gate_inp) {
    if (!m || !gate || !up || !down) return set_error(ERR_ARG, "moe_set_shared: null pointer");
    if (m->ready) return set_error(ERR_ARG, "moe_set_shared: layer already finalized");
    if (kind != KIND_Q8_0 && kind != KIND_Q4_K && kind != KIND_Q3_K)
        return set_error(ERR_QUANT_TYPE, "moe_set_shared: kind must be Q8_0, Q4_K or Q3_K");
    const size_t bg = (size_t)(row_bytes(kind, m->D) * m->F), bd = (size_t)(row_bytes(kind, m->F) * m->D);
    m->shared_kind = kind;
    if (int rc = upload_into(m->sgate, kind, m->D, m->F, gate, bg)) return rc;
    if (int rc = upload_into(m->sup, kind, m->D, m->F, up, bg)) return rc;
    if (int rc = upload_into(m->sdown, kind, m->F, m->D, down, bd)) return rc;
    if (gate_inp) {
        if (!m->sh_vec) {
            UQ_CHECK_HIP(hipMalloc(&m->sh_vec, sizeof(float) * m->D));
            m->owned.push_back(m->sh_vec);
        }
        UQ_CHECK_HIP(hipMemcpy(m->sh_vec, gate_inp, sizeof(float) * m->D, hipMemcpyHostToDevice));
    }
    m->shared_set = true;
    return OK;
}

static int moe_finalize(uq_moe* m) {
    if (m->ready) return OK;
    for (int e = 0; e < m->E; e++)
        if (!m->have[(size_t)e]) return set_error(ERR_ARG, "moe: expert " + std::to_string(e) + " not set");
    if (!m->shared_set) return set_error(ERR_ARG, "moe: shared expert not set");
    const int64_t rows_gu = (int64_t)m->F * m->E, rows_d = (int64_t)m->D * m->E;
    if (rows_gu > 4000000 || rows_d > 4000000) return set_error(ERR_SHAPE, "moe: bank too large");
    if (int rc = upload_into(m->gate, m->kind, m->D, rows_gu, m->hg.data(), m->hg.size())) return rc;
    if (int rc = upload_into(m->up, m->kind, m->D, rows_gu, m->hu.data(), m->hu.size())) return rc;
    if (int rc = upload_into(m->down, m->kind, m->F, rows_d, m->hd.data(), m->hd.size())) return rc;
    std::vector<uint8_t>().swap(m->hg);
    std::vector<uint8_t>().swap(m->hu);
    std::vector<uint8_t>().swap(m->hd);
    auto al = [&](void** p, size_t bytes) -> int {
        UQ_CHECK_HIP(hipMalloc(p, bytes));
        UQ_CHECK_HIP(hipMemsetAsync(*p, 0, bytes, (hipStream_t)uq_stream()));
        m->owned.push_back(*p);
        return OK;
    };
    const size_t slots = (size_t)m->K + 1;
    if (int rc = al((void**)&m->x, 4 * (size_t)m->D)) return rc;
    if (int rc = al((void**)&m->logits, 4 * (size_t)m->E)) return rc;
    if (int rc = al((void**)&m->out, 4 * (size_t)m->D)) return rc;
    if (int rc = al((void**)&m->xq, (size_t)m->D)) return rc;
    if (int rc = al((void**)&m->xs, 4 * (size_t)(m->D / 32))) return rc;
    if (int rc = al((void**)&m->ids, 4 * slots)) return rc;
    if (int rc = al((void**)&m->wts, 4 * slots)) return rc;
    if (int rc = al((void**)&m->status, 16)) return rc;
    if (int rc = al((void**)&m->midq, slots * m->F)) return rc;
    if (int rc = al((void**)&m->mids, 4 * slots * (m->F / 32))) return rc;
    UQ_CHECK_HIP(hipStreamSynchronize((hipStream_t)uq_stream()));
    m->ready = true;
    return OK;
}

}  // extern "C"

namespace uq {
namespace {

// NR/NS: gate/up units per lane (16 lanes per row over D); LS/DR: lanes per
// routed slot and units per lane over F in the down kernel; DS: shared-expert
// down units per lane (64 lanes over F).
template <class KR, int NR, class KS, int NS, int LS, int DR, int DS>
void moe_launch_t(const uq_moe* m, const MoeDev& d, hipStream_t s) {
    const WArgs rg{m->gate.qs, m->gate.d, m->gate.sc}, ru{m->up.qs, m->up.d, m->up.sc};
    const WArgs sg{m->sgate.qs, m->sgate.d, m->sgate.sc}, su{m->sup.qs, m->sup.d, m->sup.sc};
    const WArgs rd{m->down.qs, m->down.d, m->down.sc}, sd{m->sdown.qs, m->sdown.d, m->sdown.sc};
    hipLaunchKernelGGL((k_moe_gateup<KR, NR, KS, NS>), dim3((unsigned)((m->K + 1) * (m->F / 32))), dim3(GU_WG), 0, s,
                       d, rg, ru, sg, su);
    hipLaunchKernelGGL((k_moe_down<KR, LS, DR, KS, DS>), dim3((unsigned)((m->D + 1) / 2)), dim3(256), 0, s, d, rd,
                       sd);
}

int unit_of(uint32_t kind) { return kind == KIND_Q8_0 ? 16 : 64; }

int moe_launch(const uq_moe* m, const MoeDev& d, hipStream_t s) {
    const int D = m->D, F = m->F;
    const int nr = (D / unit_of(m->kind) + 15) / 16, ns = (D / unit_of(m->shared_kind) + 15) / 16;
    const int ndr = F / unit_of(m->kind), ds = (F / unit_of(m->shared_kind) + 63) / 64;
    // routed down row: the first (smallest) lane group in the table that holds it
#define UQ_MOE(KR, NR_, KS, NS_, LS_, DR_, DS_)                                                            \
    if (nr <= NR_ && ns <= NS_ && ndr <= LS_ * DR_ && ds <= DS_) {                                       \
        moe_launch_t<KR, NR_, KS, NS_, LS_, DR_, DS_>(m, d, s);                                             \
        return OK;                                                                                         \
    }
    if (m->kind == KIND_Q3_K && m->shared_kind == KIND_Q8_0) {
        UQ_MOE(Q3K, 1, Q8, 8, 8, 1, 1)
        UQ_MOE(Q3K, 2, Q8, 8, 8, 2, 1)
        UQ_MOE(Q3K, 2, Q8, 8, 16, 2, 2)
        UQ_MOE(Q3K, 4, Q8, 16, 32, 2, 4)
    }
    if (m->kind == KIND_Q4_K && m->shared_kind == KIND_Q8_0) {
        UQ_MOE(Q4K, 2, Q8, 8, 16, 1, 1)
        UQ_MOE(Q4K, 4, Q8, 16, 16, 1, 2)
        UQ_MOE(Q4K, 4, Q8, 16, 32, 1, 4)
        UQ_MOE(Q4K, 4, Q8, 16, 64, 1, 4)
    }
    if (m->kind == KIND_Q8_0 && m->shared_kind == KIND_Q8_0) {
        UQ_MOE(Q8, 8, Q8, 8, 64, 1, 1)
        UQ_MOE(Q8, 16, Q8, 16, 64, 4, 4)
    }
#undef UQ_MOE
    return set_error(ERR_SHAPE, "moe: unsupported kind/shape combination");
}

}  // namespace
}  // namespace uq

extern "C" {

int uq_moe_ffn_dev(uq_moe_t m, const float* x, const float* router_logits, float* out, void* stream) {
    if (!m || !x || !router_logits || !out) return set_error(ERR_ARG, "moe_ffn_dev: null pointer");
    if ((uintptr_t)x & 15) return set_error(ERR_ARG, "moe_ffn_dev: x must be 16-byte aligned");
    if (int rc = moe_finalize(m)) return rc;
    MoeDev d{x, router_logits, m->sh_vec, m->xq, m->xs, m->ids, m->wts, m->status, m->midq, m->mids, out,
             m->D, m->F, m->E, m->K};
    hipStream_t s = stream ? (hipStream_t)stream : (hipStream_t)uq_stream();
    if (int rc = moe_launch(m, d, s)) return rc;
    UQ_CHECK_HIP(hipGetLastError());
    return OK;
}

int uq_moe_run(uq_moe_t m, const float* xs, const float* logits, float* outs, int steps, double* ms) {
    if (!m || !xs || !logits || !outs || steps <= 0) return set_error(ERR_ARG, "moe_run: bad args");
    if (int rc = moe_finalize(m)) return rc;
    hipStream_t s = (hipStream_t)uq_stream();
    hipEvent_t e0, e1;
    UQ_CHECK_HIP(hipEventCreate(&e0));
    UQ_CHECK_HIP(hipEventCreate(&e1));
    UQ_CHECK_HIP(hipEventRecord(e0, s));
    for (int i = 0; i < steps; i++)
        if (int rc = uq_moe_ffn_dev(m, xs + (size_t)i * m->D, logits + (size_t)i * m->E, outs + (size_t)i * m->D, s))
            return rc;
    UQ_CHECK_HIP(hipEventRecord(e1, s));
    UQ_CHECK_HIP(hipEventSynchronize(e1));
    float t = 0;
    UQ_CHECK_HIP(hipEventElapsedTime(&t, e0, e1));
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (ms) *ms = t;
    unsigned status = 0;
    UQ_CHECK_HIP(hipMemcpy(&status, m->status, 4, hipMemcpyDeviceToHost));
    if (status) return set_error(ERR_NONFINITE, "moe_run: non-finite input in the last step");
    return OK;
}

int uq_moe_ffn(uq_moe_t m, const float* x, const float* router_logits, float* out, int32_t* ids, float* weights) {
    if (!m || !x || !router_logits || !out) return set_error(ERR_ARG, "moe_ffn: null pointer");
    if (int rc = moe_finalize(m)) return rc;
    hipStream_t s = (hipStream_t)uq_stream();
    UQ_CHECK_HIP(hipMemcpyAsync(m->x, x, 4 * (size_t)m->D, hipMemcpyHostToDevice, s));
    UQ_CHECK_HIP(hipMemcpyAsync(m->logits, router_logits, 4 * (size_t)m->E, hipMemcpyHostToDevice, s));
    if (int rc = uq_moe_ffn_dev(m, m->x, m->logits, m->out, nullptr)) return rc;
    unsigned status = 0;
    UQ_CHECK_HIP(hipMemcpyAsync(out, m->out, 4 * (size_t)m->D, hipMemcpyDeviceToHost, s));
    UQ_CHECK_HIP(hipMemcpyAsync(&status, m->status, 4, hipMemcpyDeviceToHost, s));
    if (ids) UQ_CHECK_HIP(hipMemcpyAsync(ids, m->ids, 4 * (size_t)m->K, hipMemcpyDeviceToHost, s));
    if (weights) UQ_CHECK_HIP(hipMemcpyAsync(weights, m->wts, 4 * (size_t)m->K, hipMemcpyDeviceToHost, s));
    UQ_CHECK_HIP(hipStreamSynchronize(s));
    if (status) return set_error(ERR_NONFINITE, "moe_ffn: non-finite router logits or input");
    for (int i = 0; i < m->D; i++)
        if (!std::isfinite(out[i])) return set_error(ERR_NONFINITE, "moe_ffn: non-finite output");
    return OK;
}

}  // extern "C"
