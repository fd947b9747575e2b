// MoE expert FFN for one token on gfx950: softmax routing with stable top-k,
// the selected experts' gate/up matvecs with SiLU*up and block-32 quant, their
// down matvecs and the rank-ordered weighted combine, plus the shared expert.
//
// Replaces Forward::ffn (driver/src/frontier_forward.rs:164-199) and its
// descriptor-driven multi-matvec launch (frontier_multi_matvec,
// driver/kernels/frontier_quant.cu:277-299; pack, frontier_dispatch.rs:12-31).
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

// ------------------------------------------------------------------ routing + input quant
__global__ __launch_bounds__(256) void k_moe_route(MoeDev a) {
    __shared__ float p[MAX_EXPERTS];
    __shared__ double red[4];
    __shared__ float redf[4];
    __shared__ float sum_s;
    const int t = threadIdx.x, E = a.E, D = a.D;
    unsigned bad = 0;
    // softmax: max, exp, f32 running sum in expert order (frontier_forward.rs:47-51)
    float mx = -__builtin_inff();
    for (int e = t; e < E; e += 256) {
        const float l = a.logits[e];
        bad |= !isfinite(l);
        mx = fmaxf(mx, l);
    }
    mx = block_max_f<256>(mx, redf);
    for (int e = t; e < E; e += 256) p[e] = uq_expf(a.logits[e] - mx);
    __syncthreads();
    if (t == 0) {
        float s = 0.0f;
        for (int e = 0; e < E; e++) s = s + p[e];
        sum_s = s;
    }
    __syncthreads();
    const float sum = sum_s;
    for (int e = t; e < E; e += 256) p[e] = p[e] / sum;
    __syncthreads();
    // stable top-k: rank = number of experts ordered before e
    for (int e = t; e < E; e += 256) {
        const float pe = p[e];
        int rank = 0;
        for (int j = 0; j < E; j++) rank += (p[j] > pe) || (p[j] == pe && j < e);
        if (rank < a.top_k) a.ids[rank] = e;
    }
    __syncthreads();
    // input quant (per 32) and the shared-expert gate dot in double
    double dot = 0.0;
    for (int i = t; i < D; i += 256) {
        const float v = a.x[i];
        bad |= !isfinite(v);
        if (a.sh_gate) dot = __builtin_fma((double)a.sh_gate[i], (double)v, dot);
        float s;
        const int8_t q = uq_quant_lane(v, &s);
        a.xq[i] = q;
        if ((t & 31) == 0) a.xs[i >> 5] = s;
    }
    dot = block_sum_d<256>(dot, red);
    bad = __syncthreads_or(bad);
    if (t == 0) {
        float tot = 0.0f;
        for (int k = 0; k < a.top_k; k++) tot = tot + p[a.ids[k]];
        if (!(sum > 0.0f) || !isfinite(sum) || !(tot > 0.0f)) bad = 1;
        for (int k = 0; k < a.top_k; k++) a.wts[k] = p[a.ids[k]] / tot;
        a.wts[a.top_k] = a.sh_gate ? uq_sigmoid((float)dot) : 1.0f;
        a.status[0] = bad;
    }
}

// ------------------------------------------------------------------ gate/up + SiLU + quant
// 512 threads = 32 consecutive rows of one expert's gate and up projections
// (16 lanes per row); slot < top_k is routed expert ids[slot], slot == top_k
// the shared expert. Output quantized per 32 into midq/mids[slot].
template <class KQ, int NBL>
__device__ void gateup_rows(const MoeDev& a, WArgs wg, WArgs wu, int64_t row_base, int rb, int slot, float* ys) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane & 15, grp = lane >> 4;
    const int64_t nu = a.D / KQ::UNIT;
    const int64_t row = row_base + rb * 32 + wave * 4 + grp;
    typename KQ::X xr[NBL];
    load_xr<KQ, 16, NBL>(xr, a.xq, a.xs, nu, sub);
    double g = 0.0, u = 0.0;
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int un = sub + 16 * i;
        if (un < nu) {
            g += KQ::term(wg, row, nu, un, xr[i]);
            u += KQ::term(wu, row, nu, un, xr[i]);
        }
    }
    g = uq_group_sum<16>(g);
    u = uq_group_sum<16>(u);
    if (sub == 0) {
        const float gf = (float)g, uf = (float)u;
        const float sg = gf * uq_sigmoid(gf);
        ys[wave * 4 + grp] = sg * uf;
    }
}

template <class KR, int NR, class KS, int NS>
__global__ __launch_bounds__(512) void k_moe_gateup(MoeDev a, WArgs rg, WArgs ru, WArgs sg, WArgs su) {
    __shared__ float ys[32];
    const int blocks = a.F / 32;
    const int slot = blockIdx.x / blocks, rb = blockIdx.x % blocks;
    if (slot < a.top_k) {
        const int64_t base = (int64_t)a.ids[slot] * a.F;
        gateup_rows<KR, NR>(a, rg, ru, base, rb, slot, ys);
    } else {
        gateup_rows<KS, NS>(a, sg, su, 0, rb, slot, ys);
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        const float v = ys[threadIdx.x];
        float s;
        const int8_t q = uq_quant_lane(v, &s);
        a.midq[(size_t)slot * a.F + rb * 32 + threadIdx.x] = q;
        if (threadIdx.x == 0) a.mids[(size_t)slot * (a.F / 32) + rb] = s;
    }
}

// ------------------------------------------------------------------ down + combine
// One wave per output row: each routed expert's and the shared expert's down
// row dotted with that expert's quantized mid vector, then combined in rank
// order as out = out + w*v (separate multiply and add), shared expert last.
template <class KR, int NR, class KS, int NS>
__global__ __launch_bounds__(256) void k_moe_down(MoeDev a, WArgs rd, WArgs sd) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= a.D) return;  // whole wave
    const int64_t nur = a.F / KR::UNIT, nus = a.F / KS::UNIT;
    float o = 0.0f;
    for (int k = 0; k <= a.top_k; k++) {
        const bool shared = k == a.top_k;
        double acc = 0.0;
        const int8_t* xq = a.midq + (size_t)k * a.F;
        const float* xs = a.mids + (size_t)k * (a.F / 32);
        if (!shared) {
            const int64_t r = (int64_t)a.ids[k] * a.D + row;
#pragma unroll
            for (int i = 0; i < NR; i++) {
                const int u = lane + 64 * i;
                if (u < nur) {
                    typename KR::X x;
                    KR::load_x(x, xq, xs, u);
                    acc += KR::term(rd, r, nur, u, x);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < NS; i++) {
                const int u = lane + 64 * i;
                if (u < nus) {
                    typename KS::X x;
                    KS::load_x(x, xq, xs, u);
                    acc += KS::term(sd, row, nus, u, x);
                }
            }
        }
        const float v = (float)uq_group_sum<64>(acc);
        const float tv = a.wts[k] * v;
        o = o + tv;
    }
    if (lane == 0) a.out[row] = o;
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

template <class KR, int NR, class KS, int NS, int DR, int DS>
void moe_launch_t(const uq_moe* m, const MoeDev& d, hipStream_t s) {
    const WArgs rg{m->gate.qs, m->gate.d, m->gate.sc}, ru{m->up.qs, m->up.d, m->up.sc};
    const WArgs sg{m->sgate.qs, m->sgate.d, m->sgate.sc}, su{m->sup.qs, m->sup.d, m->sup.sc};
    const WArgs rd{m->down.qs, m->down.d, m->down.sc}, sd{m->sdown.qs, m->sdown.d, m->sdown.sc};
    hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(256), 0, s, d);
    hipLaunchKernelGGL((k_moe_gateup<KR, NR, KS, NS>), dim3((unsigned)((m->K + 1) * (m->F / 32))), dim3(512), 0, s, d,
                       rg, ru, sg, su);
    hipLaunchKernelGGL((k_moe_down<KR, DR, KS, DS>), dim3((unsigned)((m->D + 3) / 4)), dim3(256), 0, s, d, rd, sd);
}

// units per lane: gate/up rows use 16 lanes over D, down rows 64 lanes over F
int moe_launch(const uq_moe* m, const MoeDev& d, hipStream_t s) {
    const int D = m->D, F = m->F;
    if (m->kind == KIND_Q3_K && m->shared_kind == KIND_Q8_0 && D == 2048 && F == 768) {
        moe_launch_t<Q3K, 1, Q8, 8, 1, 1>(m, d, s);  // D/128/16 = 1, D/16/16 = 8; F/128/64, F/16/64 <= 1
        return OK;
    }
    // general shapes: bounds on the register arrays
    const int nr = (int)((D / (m->kind == KIND_Q3_K ? 128 : m->kind == KIND_Q4_K ? 64 : 16) + 15) / 16);
    const int ns = (int)((D / (m->shared_kind == KIND_Q3_K ? 128 : m->shared_kind == KIND_Q4_K ? 64 : 16) + 15) / 16);
    const int dr = (int)((F / (m->kind == KIND_Q3_K ? 128 : m->kind == KIND_Q4_K ? 64 : 16) + 63) / 64);
    const int ds = (int)((F / (m->shared_kind == KIND_Q3_K ? 128 : m->shared_kind == KIND_Q4_K ? 64 : 16) + 63) / 64);
    if (m->kind == KIND_Q3_K && m->shared_kind == KIND_Q8_0 && nr <= 2 && ns <= 16 && dr <= 1 && ds <= 4) {
        moe_launch_t<Q3K, 2, Q8, 16, 1, 4>(m, d, s);
        return OK;
    }
    if (m->kind == KIND_Q4_K && m->shared_kind == KIND_Q8_0 && nr <= 4 && ns <= 16 && dr <= 1 && ds <= 4) {
        moe_launch_t<Q4K, 4, Q8, 16, 1, 4>(m, d, s);
        return OK;
    }
    if (m->kind == KIND_Q8_0 && m->shared_kind == KIND_Q8_0 && nr <= 16 && ns <= 16 && dr <= 4 && ds <= 4) {
        moe_launch_t<Q8, 16, Q8, 16, 4, 4>(m, d, s);
        return OK;
    }
    return set_error(ERR_SHAPE, "moe: unsupported kind/shape combination");
}

}  // namespace
}  // namespace uq

extern "C" {

int uq_moe_ffn_dev(uq_moe_t m, const float* x, const float* router_logits, float* out, void* stream) {
    if (!m || !x || !router_logits || !out) return set_error(ERR_ARG, "moe_ffn_dev: null pointer");
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
