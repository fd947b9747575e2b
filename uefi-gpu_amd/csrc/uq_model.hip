// Qwen2 dense decoder on one GPU: device-resident GGUF tensors, activation and
// fp16 KV arenas, and the decode step captured once into a hipGraph.
//
// Replaces the reference's decode graph (driver/src/gpu_graph.rs:81-197): its
// 342 prebuilt QMD jobs in one GPFIFO entry, patched per token with `token`
// and `pos`, become one hipGraphLaunch per token with `token`/`pos` read from
// device memory and the greedy result fed back on the device.
#include "uq_internal.h"
#include "uq_decode.h"
#include "uq_step.h"
#include "uq_prefill.h"
#include "uq_model.h"
#include "../../include/uq.h"

#include <cmath>
#include <cstdlib>
#include <chrono>
#include <cstring>
#include <map>
#include <string>
#include <vector>

using namespace uq;

namespace uq {

int Model::fail(int st, const std::string& msg) { return set_error(st, msg); }

const Weight* Model::weight(const std::string& name) const {
    auto it = q8.find(name);
    return it == q8.end() ? nullptr : &it->second->w;
}
const float* Model::vec(const std::string& name) const {
    auto it = f32.find(name);
    return it == f32.end() ? nullptr : it->second;
}

Model::~Model() {
    if (graph_exec) hipGraphExecDestroy(graph_exec);
    if (graph) hipGraphDestroy(graph);
    for (auto& kv : q8) uq_weight_free(kv.second);
    for (auto& kv : f32) hipFree(kv.second);
    for (auto* p : owned) hipFree(p);
    for (auto& L : layers) hipFree(L.qkv.alloc);
}

}  // namespace uq

static std::string lname(int l, const char* s) { return "blk." + std::to_string(l) + "." + s; }

extern "C" {

int uq_model_create(const uq_qwen2_config* cfg, uq_model_t* out) {
    if (!cfg || !out) return set_error(ERR_ARG, "model_create: null pointer");
    const auto& c = *cfg;
    if (c.layers <= 0 || c.dim <= 0 || c.dim % 256 || c.dim > 4096 || c.hidden <= 0 || c.hidden % 256 ||
        c.hidden > 9216 || c.heads <= 0 || c.kv_heads <= 0 || c.heads % c.kv_heads || c.head_dim % 32 ||
        c.heads * c.head_dim != c.dim || c.head_dim % 64 || c.head_dim > 256 || 1024 % c.head_dim || c.vocab <= 0 || c.max_seq <= 0 || c.max_seq > 8192)
        return set_error(ERR_SHAPE, "model_create: unsupported configuration");
    void* stream = uq_stream();
    if (!stream) return set_error(ERR_ARG, "uq_init has not been called");
    Model* m = new Model();
    m->cfg = c;
    m->stream = (hipStream_t)stream;
    *out = (uq_model_t)m;
    return OK;
}

int uq_model_free(uq_model_t h) {
    Model* m = (Model*)h;
    if (!m) return OK;
    hipStreamSynchronize(m->stream);
    delete m;
    return OK;
}

int uq_model_set_tensor(uq_model_t h, const char* name, uint32_t kind, int64_t n, int64_t rows, const void* data,
                        size_t bytes) {
    Model* m = (Model*)h;
    if (!m || !name || !data) return set_error(ERR_ARG, "model_set_tensor: null pointer");
    if (m->prepared) return set_error(ERR_ARG, "model_set_tensor: model already prepared");
    const std::string nm(name);
    if (kind == KIND_F32) {
        if (rows != 1 || n <= 0 || (int64_t)bytes != 4 * n) return set_error(ERR_SHAPE, "model_set_tensor: bad F32 shape");
        float* d = nullptr;
        UQ_CHECK_HIP(hipMalloc(&d, bytes));
        UQ_CHECK_HIP(hipMemcpy(d, data, bytes, hipMemcpyHostToDevice));
        auto it = m->f32.find(nm);
        if (it != m->f32.end()) hipFree(it->second);
        m->f32[nm] = d;
        m->f32_len[nm] = n;
        return OK;
    }
    if (kind != KIND_Q8_0) return set_error(ERR_QUANT_TYPE, "model_set_tensor: dense decoder tensors are Q8_0 or F32");
    uq_weight_t w = nullptr;
    if (int rc = uq_weight_upload(kind, n, rows, data, bytes, &w)) return rc;
    auto it = m->q8.find(nm);
    if (it != m->q8.end()) uq_weight_free(it->second);
    m->q8[nm] = w;
    return OK;
}

}  // extern "C"

namespace uq {

int Model::check_shapes() {
    const auto& c = cfg;
    const int kvd = c.kv_heads * c.head_dim;
    auto need_w = [&](const std::string& nm, int64_t n, int64_t rows) -> int {
        const Weight* w = weight(nm);
        if (!w) return fail(ERR_ARG, "missing tensor " + nm);
        if (w->n != n || w->m != rows) return fail(ERR_SHAPE, "tensor " + nm + " has the wrong shape");
        return OK;
    };
    auto need_v = [&](const std::string& nm, int64_t n, bool optional) -> int {
        auto it = f32_len.find(nm);
        if (it == f32_len.end()) return optional ? OK : fail(ERR_ARG, "missing tensor " + nm);
        if (it->second != n) return fail(ERR_SHAPE, "tensor " + nm + " has the wrong length");
        return OK;
    };
    if (int rc = need_w("token_embd.weight", c.dim, c.vocab)) return rc;
    if (int rc = need_w("output.weight", c.dim, c.vocab)) return rc;
    if (int rc = need_v("output_norm.weight", c.dim, false)) return rc;
    for (int l = 0; l < c.layers; l++) {
        if (int rc = need_w(lname(l, "attn_q.weight"), c.dim, c.dim)) return rc;
        if (int rc = need_w(lname(l, "attn_k.weight"), c.dim, kvd)) return rc;
        if (int rc = need_w(lname(l, "attn_v.weight"), c.dim, kvd)) return rc;
        if (int rc = need_w(lname(l, "attn_output.weight"), c.dim, c.dim)) return rc;
        if (int rc = need_w(lname(l, "ffn_gate.weight"), c.dim, c.hidden)) return rc;
        if (int rc = need_w(lname(l, "ffn_up.weight"), c.dim, c.hidden)) return rc;
        if (int rc = need_w(lname(l, "ffn_down.weight"), c.hidden, c.dim)) return rc;
        if (int rc = need_v(lname(l, "attn_norm.weight"), c.dim, false)) return rc;
        if (int rc = need_v(lname(l, "ffn_norm.weight"), c.dim, false)) return rc;
        if (int rc = need_v(lname(l, "attn_q.bias"), c.dim, true)) return rc;
        if (int rc = need_v(lname(l, "attn_k.bias"), kvd, true)) return rc;
        if (int rc = need_v(lname(l, "attn_v.bias"), kvd, true)) return rc;
    }
    return OK;
}

// q, k and v of a layer become one Q8_0 weight of dim + 2*kvd rows (the
// reference fuses them in one launch too, qkv_dp4a, gpu_dp4a.cu:53-59).
int Model::build_qkv(int l) {
    const Weight* ws[3] = {weight(lname(l, "attn_q.weight")), weight(lname(l, "attn_k.weight")),
                           weight(lname(l, "attn_v.weight"))};
    const int64_t n = cfg.dim, nb = n / 32;
    int64_t rows = 0;
    for (auto* w : ws) rows += w->m;
    Weight& q = layers[l].qkv;
    q.kind = KIND_Q8_0;
    q.n = n;
    q.m = rows;
    const size_t off_d = ((size_t)(n * rows) + 255) & ~(size_t)255;
    q.alloc_bytes = off_d + (((size_t)(nb * rows) * 2 + 255) & ~(size_t)255);
    UQ_CHECK_HIP(hipMalloc(&q.alloc, q.alloc_bytes));
    uint8_t* base = (uint8_t*)q.alloc;
    q.qs = (const int8_t*)base;
    q.d = (const uint16_t*)(base + off_d);
    int64_t r0 = 0;
    for (auto* w : ws) {
        UQ_CHECK_HIP(hipMemcpyAsync(base + r0 * n, w->qs, (size_t)(w->m * n), hipMemcpyDeviceToDevice, stream));
        UQ_CHECK_HIP(hipMemcpyAsync(base + off_d + r0 * nb * 2, w->d, (size_t)(w->m * nb * 2),
                                    hipMemcpyDeviceToDevice, stream));
        r0 += w->m;
    }
    UQ_CHECK_HIP(hipStreamSynchronize(stream));
    return OK;
}

template <class T>
int Model::alloc(T** p, size_t count) {
    UQ_CHECK_HIP(hipMalloc((void**)p, sizeof(T) * (count ? count : 1)));
    // zeroed on the library stream: it is non-blocking, so work queued on it is
    // not ordered after a null-stream memset
    UQ_CHECK_HIP(hipMemsetAsync(*p, 0, sizeof(T) * (count ? count : 1), stream));
    owned.push_back((void*)*p);
    return OK;
}

int Model::build_buffers() {
    const auto& c = cfg;
    const int kvd = c.kv_heads * c.head_dim;
    if (int rc = alloc(&R0, c.dim)) return rc;
    if (int rc = alloc(&R1, c.dim)) return rc;
    if (int rc = alloc(&TMP, c.dim)) return rc;
    if (int rc = alloc(&XN, c.dim)) return rc;
    if (int rc = alloc(&QKV, c.dim + 2 * kvd)) return rc;
    if (int rc = alloc(&ATT, c.dim)) return rc;
    if (int rc = alloc(&GATE, c.hidden)) return rc;
    if (int rc = alloc(&LOGITS, c.vocab)) return rc;
    if (int rc = alloc(&XQ, c.dim)) return rc;
    if (int rc = alloc(&XS, c.dim / 32)) return rc;
    if (int rc = alloc(&kcache, (size_t)c.layers * c.max_seq * kvd)) return rc;
    if (int rc = alloc(&vcache, (size_t)c.layers * c.max_seq * kvd)) return rc;
    if (int rc = alloc(&trig, (size_t)c.max_seq * c.head_dim)) return rc;
    if (int rc = alloc(&token, 1)) return rc;
    if (int rc = alloc(&pos, 1)) return rc;
    if (int rc = alloc(&history, c.max_seq)) return rc;
    if (int rc = alloc(&partial, 4 * (size_t)LM_MAX_WG)) return rc;
    if (int rc = alloc(&result, 4)) return rc;
    if (int rc = alloc(&SC, (size_t)c.heads * c.max_seq)) return rc;
    if (int rc = alloc(&CM, (size_t)c.heads * ATT_SPLIT)) return rc;
    if (int rc = alloc(&ACC, (size_t)c.heads * c.head_dim)) return rc;
    // RoPE table, gpu_graph.rs:131-133: angle = pos * powf(theta, -(2i)/hd), cos | sin
    std::vector<float> t((size_t)c.max_seq * c.head_dim);
    const int half = c.head_dim / 2;
    for (int p = 0; p < c.max_seq; p++)
        for (int i = 0; i < half; i++) {
            const float e = -((float)(2 * i)) / (float)c.head_dim;
            const float angle = (float)p * powf(c.theta, e);
            float s, co;
            sincosf(angle, &s, &co);
            t[(size_t)p * c.head_dim + i] = co;
            t[(size_t)p * c.head_dim + half + i] = s;
        }
    UQ_CHECK_HIP(hipMemcpyAsync(trig, t.data(), sizeof(float) * t.size(), hipMemcpyHostToDevice, stream));
    UQ_CHECK_HIP(hipStreamSynchronize(stream));
    return OK;
}

// One decode step, in the job order of gpu_graph.rs:137-162. The residual
// stream ping-pongs between R0 and R1: the q|k|v kernel of a layer sums
// R1 + TMP (the previous down projection) into R0, the gate/up kernel sums
// R0 + TMP (the o projection) into R1.
int Model::enqueue_step(hipStream_t s) {
    const auto& c = cfg;
    const int kvd = c.kv_heads * c.head_dim;
    const size_t kvl = (size_t)c.max_seq * kvd;
    const Weight* emb = weight("token_embd.weight");
    auto nq_args = [&](const float* xin, const float* res, const float* gamma, float* xout) {
        NormQuantArgs nq{};
        nq.x = xin;
        nq.residual = res;
        nq.gamma = gamma;
        nq.x_out = xout;
        nq.dim = c.dim;
        nq.eps = c.eps;
        return nq;
    };
    for (int l = 0; l < c.layers; l++) {
        const Weight& qkv = layers[l].qkv;
        NormQuantArgs na = nq_args(R1, TMP, vec(lname(l, "attn_norm.weight")), R0);
        if (l == 0) {
            na.embed_qs = emb->qs;
            na.embed_d = emb->d;
            na.token = token;
        }
        QkvArgs qa{qkv.qs, qkv.d, na, vec(lname(l, "attn_q.bias")), vec(lname(l, "attn_k.bias")),
                   vec(lname(l, "attn_v.bias")), trig, pos, QKV, kcache + l * kvl, vcache + l * kvl,
                   c.dim, c.heads, c.kv_heads, c.head_dim};
        if (launch_qkv_rope(qa, s)) return fail(ERR_SHAPE, "qkv_rope: unsupported dim");
        AttSplitArgs aa{QKV, kcache + l * kvl, vcache + l * kvl, pos, SC, CM, ACC, c.heads, c.kv_heads, c.head_dim,
                        c.max_seq, (float)(1.0 / std::sqrt((double)c.head_dim))};
        if (launch_attention_split(aa, s)) return fail(ERR_SHAPE, "attention: head_dim / max_seq beyond the LDS budget");
        const Weight* wo = weight(lname(l, "attn_output.weight"));
        WoArgs wa{wo->qs, wo->d, ACC, TMP, wo->m, wo->n};
        if (launch_wo_acc(wa, s)) return fail(ERR_SHAPE, "o projection: unsupported dim");
        const Weight *wg = weight(lname(l, "ffn_gate.weight")), *wu = weight(lname(l, "ffn_up.weight"));
        GateArgs ga{wg->qs, wu->qs, wg->d, wu->d, nq_args(R0, TMP, vec(lname(l, "ffn_norm.weight")), R1), GATE,
                    c.hidden, c.dim};
        if (launch_gateup_h(ga, s)) return fail(ERR_SHAPE, "gate/up: unsupported dim");
        const Weight* wd = weight(lname(l, "ffn_down.weight"));
        DownArgs da{wd->qs, wd->d, GATE, TMP, wd->m, wd->n};
        if (launch_down_h(da, s)) return fail(ERR_SHAPE, "down: unsupported hidden size");
    }
    const Weight* out = weight("output.weight");
    LmArgs la{out->qs, out->d, XQ, XS, LOGITS, c.vocab, c.dim, partial, result, token, pos, history, c.max_seq};
    la.nq = nq_args(R1, TMP, vec("output_norm.weight"), nullptr);  // the output norm runs inside the lm_head launch
    if (launch_lm_greedy(la, s)) return fail(ERR_SHAPE, "lm_head: unsupported dim");
    return OK;
}

int Model::prepare() {
    if (prepared) return OK;
    if (int rc = check_shapes()) return rc;
    layers.resize(cfg.layers);
    for (int l = 0; l < cfg.layers; l++) {
        if (int rc = build_qkv(l)) return rc;
        for (const char* s : {"attn_q.weight", "attn_k.weight", "attn_v.weight"}) {
            auto it = q8.find(lname(l, s));
            uq_weight_free(it->second);
            q8.erase(it);
        }
    }
    if (int rc = build_buffers()) return rc;
    if (int rc = build_prefill()) return rc;
    UQ_CHECK_HIP(hipStreamSynchronize(stream));
    // UQ_DECODE_EAGER=1 launches the step's kernels directly instead of through
    // the captured graph (same kernels and order; used to profile per kernel).
    const char* eager_env = getenv("UQ_DECODE_EAGER");
    eager = eager_env && eager_env[0] == '1';
    if (eager) {
        prepared = true;
        return OK;
    }
    UQ_CHECK_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_step(stream);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(stream, &g);
    if (rc) {
        if (g) hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return fail(ERR_DEVICE, std::string("graph capture: ") + hipGetErrorString(e));
    graph = g;
    UQ_CHECK_HIP(hipGraphInstantiate(&graph_exec, graph, nullptr, nullptr, 0));
    prepared = true;
    return OK;
}

// Prefill arenas and the transposed weight scales of every layer.
int Model::build_prefill() {
    const auto& c = cfg;
    const int kvd = c.kv_heads * c.head_dim, nqkv = c.dim + 2 * kvd;
    const int cap = c.max_seq < 1024 ? c.max_seq : 1024;
    pcap = (cap + 63) / 64 * 64;
    const int big = c.hidden > nqkv ? c.hidden : nqkv;
    if (int rc = alloc(&PX, (size_t)pcap * c.dim)) return rc;
    if (int rc = alloc(&PTMP, (size_t)pcap * c.dim)) return rc;
    if (int rc = alloc(&PY, (size_t)pcap * nqkv)) return rc;
    if (int rc = alloc(&PATT, (size_t)pcap * c.dim)) return rc;
    if (int rc = alloc(&PG, (size_t)pcap * c.hidden)) return rc;
    if (int rc = alloc(&PXQ, (size_t)pcap * big)) return rc;
    if (int rc = alloc(&PXST, (size_t)pcap * big / 32)) return rc;
    if (int rc = alloc(&PTOK, (size_t)pcap)) return rc;
    auto tr = [&](const Weight& w, float** dt) -> int {
        if (int rc = alloc(dt, (size_t)w.m * (w.n / 32))) return rc;
        launch_transpose_scales(w.d, w.m, w.n / 32, *dt, stream);
        return OK;
    };
    // q|k|v row order of the prefill copy: within each q and k head, row 2j + e
    // = output j + e * hd/2 (the RoPE pair adjacent); v unchanged
    std::vector<int> perm((size_t)nqkv);
    const int hd = c.head_dim, half = hd / 2;
    for (int r = 0; r < nqkv; r++) {
        if (r < c.dim + kvd) {
            const int base = r < c.dim ? 0 : c.dim, w = r - base;
            perm[r] = base + (w / hd) * hd + (w % hd) / 2 + (w % 2) * half;
        } else {
            perm[r] = r;
        }
    }
    int* dperm = nullptr;
    if (int rc = alloc(&dperm, (size_t)nqkv)) return rc;
    UQ_CHECK_HIP(hipMemcpyAsync(dperm, perm.data(), 4 * (size_t)nqkv, hipMemcpyHostToDevice, stream));
    float *dt_tmp = nullptr, *bias_tmp = nullptr;
    if (int rc = alloc(&dt_tmp, (size_t)nqkv * (c.dim / 32))) return rc;
    if (int rc = alloc(&bias_tmp, (size_t)nqkv)) return rc;
    for (int l = 0; l < c.layers; l++) {
        LayerDev& L = layers[l];
        launch_transpose_scales(L.qkv.d, L.qkv.m, L.qkv.n / 32, dt_tmp, stream);
        if (int rc = alloc(&L.qkv_dt, (size_t)nqkv * (c.dim / 32))) return rc;
        launch_gather_cols(dt_tmp, c.dim / 32, nqkv, dperm, L.qkv_dt, stream);
        if (int rc = alloc(&L.qkv_pq, (size_t)nqkv * c.dim)) return rc;
        launch_gather_rows(L.qkv.qs, c.dim, dperm, nqkv, L.qkv_pq, stream);
        const char* bn[3] = {"attn_q.bias", "attn_k.bias", "attn_v.bias"};
        const int boff[3] = {0, c.dim, c.dim + kvd}, blen[3] = {c.dim, kvd, kvd};
        for (int i = 0; i < 3; i++) {
            const float* b = vec(lname(l, bn[i]));
            if (b) UQ_CHECK_HIP(hipMemcpyAsync(bias_tmp + boff[i], b, 4 * (size_t)blen[i], hipMemcpyDeviceToDevice, stream));
            else UQ_CHECK_HIP(hipMemsetAsync(bias_tmp + boff[i], 0, 4 * (size_t)blen[i], stream));
        }
        if (int rc = alloc(&L.qkv_pb, (size_t)nqkv)) return rc;
        launch_gather_cols(bias_tmp, 1, nqkv, dperm, L.qkv_pb, stream);
        if (int rc = tr(*weight(lname(l, "attn_output.weight")), &L.o_dt)) return rc;
        if (int rc = tr(*weight(lname(l, "ffn_gate.weight")), &L.g_dt)) return rc;
        if (int rc = tr(*weight(lname(l, "ffn_up.weight")), &L.u_dt)) return rc;
        if (int rc = tr(*weight(lname(l, "ffn_down.weight")), &L.d_dt)) return rc;
    }
    UQ_CHECK_HIP(hipGetLastError());
    UQ_CHECK_HIP(hipStreamSynchronize(stream));
    return OK;
}

// Prompt prefill at positions 0..n-1 in the job order of prepare_prefill
// (gpu_prefill.rs:122-150): per layer norm+quant, q|k|v GEMM, RoPE + KV,
// causal attention, quant, o GEMM, norm+quant, gate/up GEMM with SiLU, quant,
// down GEMM; then the last token's residual through the decode output head.
int Model::prefill(const uint32_t* tokens, int n, uint32_t* next) {
    const auto& c = cfg;
    if (n <= 0 || n > pcap || n > c.max_seq) return fail(ERR_CONTEXT, "prefill: prompt longer than the prefill window");
    for (int i = 0; i < n; i++)
        if ((int64_t)tokens[i] >= c.vocab) return fail(ERR_SHAPE, "prefill: token id beyond the vocabulary");
    const int kvd = c.kv_heads * c.head_dim, nqkv = c.dim + 2 * kvd;
    const int mp = (n + 63) / 64 * 64;
    const size_t kvl = (size_t)c.max_seq * kvd;
    const hipStream_t s = stream;
    const Weight* emb = weight("token_embd.weight");
    UQ_CHECK_HIP(hipMemcpyAsync(PTOK, tokens, 4 * (size_t)n, hipMemcpyHostToDevice, s));
    auto norm = [&](int l, const float* gamma, bool first) {
        PfNormArgs na{};
        na.nq.gamma = gamma;
        na.nq.dim = c.dim;
        na.nq.eps = c.eps;
        if (first) {
            na.nq.embed_qs = emb->qs;
            na.nq.embed_d = emb->d;
            na.tokens = PTOK;
        } else {
            na.residual = PTMP;
        }
        na.x = PX;
        na.xq = PXQ;
        na.xst = PXST;
        na.mp = mp;
        launch_pf_norm(na, n, s);
    };
    // the gate/up GEMM quantizes SiLU(gate)*up into the arena of PG (codes,
    // then scales) for the down GEMM
    int8_t* const hq = (int8_t*)PG;
    float* const hst = (float*)((char*)PG + (((size_t)pcap * c.hidden + 255) & ~(size_t)255));
    auto gemm = [&](const Weight& w, const float* dt, const Weight* w2, const float* dt2, float* y,
                    const int8_t* xq = nullptr, const float* xst = nullptr, int8_t* yq = nullptr, float* yst = nullptr) {
        PfGemmArgs ga{w.qs, dt, w2 ? w2->qs : nullptr, dt2, xq ? xq : PXQ, xst ? xst : PXST, y, w.m, w.n, mp, yq, yst};
        return launch_pf_gemm(ga, s);
    };
    for (int l = 0; l < c.layers; l++) {
        const LayerDev& L = layers[l];
        norm(l, vec(lname(l, "attn_norm.weight")), l == 0);
        {
            // q|k|v GEMM on the permuted copy with the bias + RoPE + KV epilogue
            PfGemmArgs ga{L.qkv_pq, L.qkv_dt, nullptr, nullptr, PXQ, PXST, PY, L.qkv.m, L.qkv.n, mp, nullptr, nullptr};
            ga.rope = 1;
            ga.re = PfRopeEpi{PY, nqkv, L.qkv_pb, vec(lname(l, "attn_q.bias")) != nullptr,
                              vec(lname(l, "attn_k.bias")) != nullptr, vec(lname(l, "attn_v.bias")) != nullptr, trig,
                              kcache + l * kvl, vcache + l * kvl, n, 0, c.heads, c.kv_heads, c.head_dim};
            if (launch_pf_gemm(ga, s)) return fail(ERR_SHAPE, "prefill: q|k|v rows not a multiple of 64");
        }
        // head_dim 128: the attention epilogue quantizes its output for the o GEMM
        const bool fused_quant = c.head_dim == 128;
        PfAttnArgs aa{PY, nqkv, kcache + l * kvl, vcache + l * kvl, PATT, n, 0, c.max_seq, c.heads, c.kv_heads, c.head_dim,
                      (float)(1.0 / std::sqrt((double)c.head_dim)), fused_quant ? PXQ : nullptr,
                      fused_quant ? PXST : nullptr, mp};
        if (launch_pf_attention(aa, s)) return fail(ERR_SHAPE, "prefill: attention head_dim unsupported");
        if (!fused_quant) launch_pf_quant(PATT, c.dim, n, mp, PXQ, PXST, s);
        if (gemm(*weight(lname(l, "attn_output.weight")), L.o_dt, nullptr, nullptr, PTMP))
            return fail(ERR_SHAPE, "prefill: o rows not a multiple of 64");
        norm(l, vec(lname(l, "ffn_norm.weight")), false);
        if (gemm(*weight(lname(l, "ffn_gate.weight")), L.g_dt, weight(lname(l, "ffn_up.weight")), L.u_dt, nullptr,
                 nullptr, nullptr, hq, hst))
            return fail(ERR_SHAPE, "prefill: ffn rows not a multiple of 64");
        if (gemm(*weight(lname(l, "ffn_down.weight")), L.d_dt, nullptr, nullptr, PTMP, hq, hst))
            return fail(ERR_SHAPE, "prefill: down rows not a multiple of 64");
    }
    // the last prompt token through the decode output head (gpu_prefill.rs:138-148)
    NormQuantArgs no{};
    no.x = PX + (size_t)(n - 1) * c.dim;
    no.residual = PTMP + (size_t)(n - 1) * c.dim;
    no.gamma = vec("output_norm.weight");
    no.dim = c.dim;
    no.eps = c.eps;
    host_io[1] = (uint32_t)(n - 1);
    UQ_CHECK_HIP(hipMemcpyAsync(pos, &host_io[1], 4, hipMemcpyHostToDevice, s));
    const Weight* out = weight("output.weight");
    LmArgs la{out->qs, out->d, XQ, XS, LOGITS, c.vocab, c.dim, partial, result, token, pos, history, c.max_seq};
    la.nq = no;  // the output norm runs inside the lm_head launch
    if (launch_lm_greedy(la, s)) return fail(ERR_SHAPE, "lm_head: unsupported dim");
    UQ_CHECK_HIP(hipGetLastError());
    uint32_t res[2] = {0, 0};
    UQ_CHECK_HIP(hipMemcpyAsync(res, result, 8, hipMemcpyDeviceToHost, s));
    UQ_CHECK_HIP(hipStreamSynchronize(s));
    if (res[1]) return fail(ERR_NONFINITE, "prefill: non-finite logits");
    *next = res[0];
    return OK;
}

int Model::launch_step() {
    if (eager) return enqueue_step(stream);
    UQ_CHECK_HIP(hipGraphLaunch(graph_exec, stream));
    return OK;
}

int Model::set_position(uint32_t tok, int p) {
    if ((int64_t)tok >= cfg.vocab) return fail(ERR_SHAPE, "token id beyond the vocabulary");
    if (p < 0 || p >= cfg.max_seq) return fail(ERR_CONTEXT, "position beyond the KV cache");
    host_io[0] = tok;
    host_io[1] = (uint32_t)p;
    UQ_CHECK_HIP(hipMemcpyAsync(token, &host_io[0], 4, hipMemcpyHostToDevice, stream));
    UQ_CHECK_HIP(hipMemcpyAsync(pos, &host_io[1], 4, hipMemcpyHostToDevice, stream));
    return OK;
}

}  // namespace uq

extern "C" {

int uq_model_prepare(uq_model_t h) {
    Model* m = (Model*)h;
    if (!m) return set_error(ERR_ARG, "model_prepare: null model");
    return m->prepare();
}

int uq_decode_step(uq_model_t h, uint32_t tok, int p, uint32_t* next) {
    Model* m = (Model*)h;
    if (!m || !next) return set_error(ERR_ARG, "decode_step: null pointer");
    if (!m->prepared) return set_error(ERR_ARG, "decode_step: model not prepared");
    if (int rc = m->set_position(tok, p)) return rc;
    if (int rc = m->launch_step()) return rc;
    uint32_t res[2] = {0, 0};
    UQ_CHECK_HIP(hipMemcpyAsync(res, m->result, 8, hipMemcpyDeviceToHost, m->stream));
    UQ_CHECK_HIP(hipStreamSynchronize(m->stream));
    if (res[1]) return set_error(ERR_NONFINITE, "decode_step: non-finite logits");
    if ((int64_t)res[0] >= m->cfg.vocab) return set_error(ERR_DEVICE, "decode_step: invalid token id");
    *next = res[0];
    return OK;
}

int uq_decode_run(uq_model_t h, uint32_t tok, int p, int steps, uint32_t* tokens, double* ms) {
    Model* m = (Model*)h;
    if (!m || !tokens) return set_error(ERR_ARG, "decode_run: null pointer");
    if (!m->prepared) return set_error(ERR_ARG, "decode_run: model not prepared");
    if (steps <= 0 || p < 0 || (int64_t)p + steps > m->cfg.max_seq)
        return set_error(ERR_CONTEXT, "decode_run: positions beyond the KV cache");
    if (int rc = m->set_position(tok, p)) return rc;
    UQ_CHECK_HIP(hipMemsetAsync(m->result + 2, 0, 4, m->stream));
    hipEvent_t e0, e1;
    UQ_CHECK_HIP(hipEventCreate(&e0));
    UQ_CHECK_HIP(hipEventCreate(&e1));
    UQ_CHECK_HIP(hipEventRecord(e0, m->stream));
    for (int i = 0; i < steps; i++)
        if (int rc = m->launch_step()) return rc;
    UQ_CHECK_HIP(hipEventRecord(e1, m->stream));
    std::vector<uint32_t> out((size_t)steps);
    uint32_t res[3] = {0, 0, 0};
    UQ_CHECK_HIP(hipMemcpyAsync(out.data(), m->history + p, 4 * (size_t)steps, hipMemcpyDeviceToHost, m->stream));
    UQ_CHECK_HIP(hipMemcpyAsync(res, m->result, 12, hipMemcpyDeviceToHost, m->stream));
    UQ_CHECK_HIP(hipStreamSynchronize(m->stream));
    float t = 0;
    hipEventElapsedTime(&t, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (ms) *ms = t;
    std::memcpy(tokens, out.data(), 4 * (size_t)steps);
    if (res[2]) return set_error(ERR_NONFINITE, "decode_run: non-finite logits");
    return OK;
}

int uq_prompt_tokens(uq_model_t h, const uint32_t* tokens, int count, int p, uint32_t* next) {
    Model* m = (Model*)h;
    if (!m || !tokens || !next) return set_error(ERR_ARG, "prompt_tokens: null pointer");
    if (!m->prepared) return set_error(ERR_ARG, "prompt_tokens: model not prepared");
    if (count <= 0 || p < 0 || (int64_t)p + count > m->cfg.max_seq)
        return set_error(ERR_CONTEXT, "prompt_tokens: positions beyond the KV cache");
    for (int i = 0; i < count; i++)
        if ((int64_t)tokens[i] >= m->cfg.vocab) return set_error(ERR_SHAPE, "prompt_tokens: token id beyond the vocabulary");
    std::vector<uint32_t> staged(tokens, tokens + count);
    for (int i = 0; i < count; i++) {
        const int pp = p + i;
        UQ_CHECK_HIP(hipMemcpyAsync(m->token, &staged[i], 4, hipMemcpyHostToDevice, m->stream));
        UQ_CHECK_HIP(hipMemcpyAsync(m->pos, &pp, 4, hipMemcpyHostToDevice, m->stream));
        if (int rc = m->launch_step()) return rc;
        UQ_CHECK_HIP(hipStreamSynchronize(m->stream));
    }
    uint32_t res[2] = {0, 0};
    UQ_CHECK_HIP(hipMemcpyAsync(res, m->result, 8, hipMemcpyDeviceToHost, m->stream));
    UQ_CHECK_HIP(hipStreamSynchronize(m->stream));
    if (res[1]) return set_error(ERR_NONFINITE, "prompt_tokens: non-finite logits");
    *next = res[0];
    return OK;
}

int uq_prefill(uq_model_t h, const uint32_t* tokens, int count, uint32_t* next) {
    Model* m = (Model*)h;
    if (!m || !tokens || !next) return set_error(ERR_ARG, "prefill: null pointer");
    if (!m->prepared) return set_error(ERR_ARG, "prefill: model not prepared");
    return m->prefill(tokens, count, next);
}

// generate_one (driver/src/llm.rs:402-428): the prompt through the prefill,
// then greedy steps. Before each step the current id is checked against the
// stop ids (end of generation); otherwise it is appended to the output and fed
// to the next step at position count + i. Host clock per phase, each phase
// ending with its result on the host.
int uq_generate(uq_model_t h, const uint32_t* prompt, int count, int max_new, const uint32_t* stop, int nstop,
                uint32_t* out, int* generated, int* ended, double* prefill_ms, double* decode_ms) {
    Model* m = (Model*)h;
    if (!m || !prompt || !out || !generated || !ended || (nstop > 0 && !stop))
        return set_error(ERR_ARG, "generate: null pointer");
    if (!m->prepared) return set_error(ERR_ARG, "generate: model not prepared");
    if (count <= 0 || max_new < 0 || (int64_t)count + max_new >= m->cfg.max_seq)
        return set_error(ERR_CONTEXT, "generate: prompt + new tokens must stay below max_seq");
    auto is_stop = [&](uint32_t t) {
        for (int k = 0; k < nstop; k++)
            if (stop[k] == t) return true;
        return false;
    };
    using clk = std::chrono::steady_clock;
    const auto t0 = clk::now();
    uint32_t next = 0;
    if (int rc = m->prefill(prompt, count, &next)) return rc;
    const auto t1 = clk::now();
    int n = 0;
    bool end = false;
    for (int i = 0; i < max_new; i++) {
        if (is_stop(next)) {
            end = true;
            break;
        }
        out[n++] = next;
        if (int rc = uq_decode_step(h, next, count + i, &next)) return rc;
    }
    if (is_stop(next)) end = true;
    const auto t2 = clk::now();
    *generated = n;
    *ended = end ? 1 : 0;
    if (prefill_ms) *prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (decode_ms) *decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
    return OK;
}

int uq_prefill_gemm(uq_weight_t w, const int8_t* xq, const float* xs, int64_t tokens, float* y) {
    if (!w || !xq || !xs || !y) return set_error(ERR_ARG, "prefill_gemm: null pointer");
    const Weight& W = w->w;
    if (W.kind != KIND_Q8_0) return set_error(ERR_QUANT_TYPE, "prefill_gemm: Q8_0 only");
    if (W.m % 64 || tokens <= 0 || tokens > 4096) return set_error(ERR_SHAPE, "prefill_gemm: rows % 64, 1..4096 tokens");
    hipStream_t s = (hipStream_t)uq_stream();
    const int64_t k = W.n, nb = k / 32, mp = (tokens + 63) / 64 * 64;
    std::vector<float> xst((size_t)(nb * mp), 0.0f);
    for (int64_t t = 0; t < tokens; t++)
        for (int64_t b = 0; b < nb; b++) xst[b * mp + t] = xs[t * nb + b];
    float* dt = nullptr;
    int8_t* dq = nullptr;
    float *ds = nullptr, *dy = nullptr;
    UQ_CHECK_HIP(hipMalloc(&dt, 4 * (size_t)(nb * W.m)));
    UQ_CHECK_HIP(hipMalloc(&dq, (size_t)(mp * k)));
    UQ_CHECK_HIP(hipMalloc(&ds, 4 * xst.size()));
    UQ_CHECK_HIP(hipMalloc(&dy, 4 * (size_t)(mp * W.m)));
    UQ_CHECK_HIP(hipMemsetAsync(dq, 0, (size_t)(mp * k), s));
    UQ_CHECK_HIP(hipMemcpyAsync(dq, xq, (size_t)(tokens * k), hipMemcpyHostToDevice, s));
    UQ_CHECK_HIP(hipMemcpyAsync(ds, xst.data(), 4 * xst.size(), hipMemcpyHostToDevice, s));
    launch_transpose_scales(W.d, W.m, nb, dt, s);
    PfGemmArgs ga{W.qs, dt, nullptr, nullptr, dq, ds, dy, W.m, k, (int)mp};
    int rc = launch_pf_gemm(ga, s) ? set_error(ERR_SHAPE, "prefill_gemm: shape") : OK;
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && rc == OK) e = hipMemcpyAsync(y, dy, 4 * (size_t)(tokens * W.m), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    hipFree(dt);
    hipFree(dq);
    hipFree(ds);
    hipFree(dy);
    if (e != hipSuccess) return set_error(ERR_DEVICE, std::string("prefill_gemm: ") + hipGetErrorString(e));
    return rc;
}

int uq_time_prefill_gemm(uq_weight_t w, uq_weight_t w2, int64_t tokens, int reps, double* ms) {
    if (!w || reps <= 0 || !ms) return set_error(ERR_ARG, "time_prefill_gemm: bad args");
    const Weight& W = w->w;
    if (W.kind != KIND_Q8_0 || W.m % 64 || tokens <= 0 || tokens > 4096)
        return set_error(ERR_SHAPE, "time_prefill_gemm: Q8_0, rows % 64, 1..4096 tokens");
    if (w2 && (w2->w.m != W.m || w2->w.n != W.n)) return set_error(ERR_SHAPE, "time_prefill_gemm: pair shapes differ");
    hipStream_t s = (hipStream_t)uq_stream();
    const int64_t k = W.n, nb = k / 32, mp = (tokens + 63) / 64 * 64;
    std::vector<int8_t> hq((size_t)(mp * k));
    std::vector<float> hs((size_t)(nb * mp));
    for (size_t i = 0; i < hq.size(); i++) hq[i] = (int8_t)((int)((i * 2654435761u) >> 24) % 255 - 127);
    for (size_t i = 0; i < hs.size(); i++) hs[i] = 0.01f + 0.001f * (float)(i % 7);
    float *dt = nullptr, *dt2 = nullptr;
    int8_t* dq = nullptr;
    float *ds = nullptr, *dy = nullptr;
    UQ_CHECK_HIP(hipMalloc(&dt, 4 * (size_t)(nb * W.m)));
    if (w2) UQ_CHECK_HIP(hipMalloc(&dt2, 4 * (size_t)(nb * W.m)));
    UQ_CHECK_HIP(hipMalloc(&dq, hq.size()));
    UQ_CHECK_HIP(hipMalloc(&ds, 4 * hs.size()));
    UQ_CHECK_HIP(hipMalloc(&dy, 4 * (size_t)(mp * W.m)));
    UQ_CHECK_HIP(hipMemcpyAsync(dq, hq.data(), hq.size(), hipMemcpyHostToDevice, s));
    UQ_CHECK_HIP(hipMemcpyAsync(ds, hs.data(), 4 * hs.size(), hipMemcpyHostToDevice, s));
    launch_transpose_scales(W.d, W.m, nb, dt, s);
    if (w2) launch_transpose_scales(w2->w.d, W.m, nb, dt2, s);
    PfGemmArgs ga{W.qs, dt, w2 ? w2->w.qs : nullptr, dt2, dq, ds, dy, W.m, k, (int)mp};
    hipEvent_t e0, e1;
    UQ_CHECK_HIP(hipEventCreate(&e0));
    UQ_CHECK_HIP(hipEventCreate(&e1));
    int rc = launch_pf_gemm(ga, s) ? set_error(ERR_SHAPE, "time_prefill_gemm: shape") : OK;
    if (rc == OK) {
        UQ_CHECK_HIP(hipEventRecord(e0, s));
        for (int r = 0; r < reps; r++) launch_pf_gemm(ga, s);
        UQ_CHECK_HIP(hipEventRecord(e1, s));
        UQ_CHECK_HIP(hipEventSynchronize(e1));
        float t = 0;
        UQ_CHECK_HIP(hipEventElapsedTime(&t, e0, e1));
        *ms = t / reps;
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipFree(dt);
    if (dt2) hipFree(dt2);
    hipFree(dq);
    hipFree(ds);
    hipFree(dy);
    return rc;
}

int uq_time_prefill_attention(int32_t tokens, int32_t heads, int32_t kv_heads, int32_t head_dim, int quant_out,
                              int reps, double* ms) {
    if (reps <= 0 || !ms || tokens <= 0 || tokens > 1024 || heads <= 0 || kv_heads <= 0 || heads % kv_heads ||
        (head_dim != 64 && head_dim != 128) || (quant_out && head_dim != 128))
        return set_error(ERR_ARG, "time_prefill_attention: bad args");
    hipStream_t s = (hipStream_t)uq_stream();
    const int64_t stride = (int64_t)(heads + 2 * kv_heads) * head_dim, kvd = (int64_t)kv_heads * head_dim;
    const int64_t qd = (int64_t)heads * head_dim, mp = (tokens + 63) / 64 * 64;
    // q rows in [-1, 1); fp16 keys and values of magnitude [1/4, 2), random sign
    std::vector<float> hq((size_t)(tokens * stride));
    for (size_t i = 0; i < hq.size(); i++) hq[i] = (float)((int)((i * 2654435761u) >> 16) % 2048 - 1024) / 1024.0f;
    std::vector<uint16_t> hkv((size_t)(2 * tokens * kvd));
    for (size_t i = 0; i < hkv.size(); i++) {
        const uint32_t r = (uint32_t)((i + 1) * 2246822519u) >> 7;
        hkv[i] = (uint16_t)(((r >> 20) & 1) << 15 | (13 + (r >> 10) % 3) << 10 | (r & 0x3ff));
    }
    float *dq = nullptr, *dout = nullptr, *dxs = nullptr;
    uint16_t* dkv = nullptr;
    int8_t* dxq = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipMalloc(&dq, 4 * hq.size());
    if (e == hipSuccess) e = hipMalloc(&dkv, 2 * hkv.size());
    if (e == hipSuccess) e = hipMalloc(&dout, 4 * (size_t)(tokens * qd));
    if (e == hipSuccess) e = hipMalloc(&dxq, (size_t)(mp * qd));
    if (e == hipSuccess) e = hipMalloc(&dxs, 4 * (size_t)(qd / 32 * mp));
    if (e == hipSuccess) e = hipMemcpyAsync(dq, hq.data(), 4 * hq.size(), hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(dkv, hkv.data(), 2 * hkv.size(), hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    int rc = OK;
    if (e == hipSuccess) {
        PfAttnArgs aa{dq, (int)stride, dkv, dkv + tokens * kvd, dout, tokens, 0, tokens, heads, kv_heads, head_dim,
                      (float)(1.0 / std::sqrt((double)head_dim)), quant_out ? dxq : nullptr, quant_out ? dxs : nullptr,
                      (int)mp};
        if (launch_pf_attention(aa, s)) {
            rc = set_error(ERR_SHAPE, "time_prefill_attention: shape");
        } else {
            e = hipEventRecord(e0, s);
            for (int r = 0; r < reps && e == hipSuccess; r++) e = launch_pf_attention(aa, s) ? hipErrorInvalidValue : hipSuccess;
            if (e == hipSuccess) e = hipEventRecord(e1, s);
            if (e == hipSuccess) e = hipEventSynchronize(e1);
            float t = 0;
            if (e == hipSuccess) e = hipEventElapsedTime(&t, e0, e1);
            *ms = t / reps;
        }
    }
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    hipFree(dq);
    hipFree(dkv);
    hipFree(dout);
    hipFree(dxq);
    hipFree(dxs);
    if (e != hipSuccess) return set_error(ERR_DEVICE, std::string("time_prefill_attention: ") + hipGetErrorString(e));
    return rc;
}

int uq_model_logits(uq_model_t h, float* out, int64_t n) {
    Model* m = (Model*)h;
    if (!m || !out) return set_error(ERR_ARG, "model_logits: null pointer");
    if (!m->prepared) return set_error(ERR_ARG, "model_logits: model not prepared");
    if (n != m->cfg.vocab) return set_error(ERR_SHAPE, "model_logits: n != vocab");
    UQ_CHECK_HIP(hipMemcpyAsync(out, m->LOGITS, 4 * (size_t)n, hipMemcpyDeviceToHost, m->stream));
    UQ_CHECK_HIP(hipStreamSynchronize(m->stream));
    return OK;
}

int uq_model_kv(uq_model_t h, int layer, int count, uint16_t* keys, uint16_t* values) {
    Model* m = (Model*)h;
    if (!m || !keys || !values) return set_error(ERR_ARG, "model_kv: null pointer");
    if (!m->prepared) return set_error(ERR_ARG, "model_kv: model not prepared");
    if (layer < 0 || layer >= m->cfg.layers || count <= 0 || count > m->cfg.max_seq)
        return set_error(ERR_SHAPE, "model_kv: bad layer or count");
    const size_t kvd = (size_t)m->cfg.kv_heads * m->cfg.head_dim, kvl = kvd * m->cfg.max_seq;
    UQ_CHECK_HIP(hipMemcpyAsync(keys, m->kcache + layer * kvl, 2 * kvd * count, hipMemcpyDeviceToHost, m->stream));
    UQ_CHECK_HIP(hipMemcpyAsync(values, m->vcache + layer * kvl, 2 * kvd * count, hipMemcpyDeviceToHost, m->stream));
    UQ_CHECK_HIP(hipStreamSynchronize(m->stream));
    return OK;
}

}  // extern "C"
