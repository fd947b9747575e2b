// Decode-step kernels for gfx950 besides the matvecs: embedding + residual +
// RMSNorm + block-32 quant, q/k bias + RoPE + fp16 KV write, GQA attention over
// the fp16 cache with the output quantized in place, and greedy selection.
//
// Reference kernels replaced: embedding_q8 (gpu_embedding.cu:298-304),
// fused_resnorm / fused_resnorm_quant (gpu_fused.cu:193-200,
// gpu_norm_quant.cu:307-323), quant_act (gpu_dp4a.cu:23-31), rope_bias
// (gpu_ops.cu:235-246), fused_attention (gpu_attention.cu:202-226),
// greedy_tiles / greedy_finish (gpu_greedy.cu:269-295).
//
// Position and token live in device memory so that one captured graph serves
// every step (the reference patches them into its push buffer per token,
// gpu_graph.rs:170-178).
#include "uq_device.h"
#include "uq_decode.h"

namespace uq {
namespace {

// Sum of a double over the whole workgroup (WG threads, multiple of 64).
template <int WG>
__device__ double block_sum_d(double v, double* red) {
    v = uq_group_sum<64>(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < WG / 64; w++) t += red[w];
    return t;
}
template <int WG>
__device__ float block_max_f(float v, float* red) {
    v = uq_group_max<64>(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int w = 1; w < WG / 64; w++) t = fmaxf(t, red[w]);
    return t;
}

constexpr int NQ_WG = 256;
constexpr int NQ_MAX_PER_THREAD = 16;  // dim <= 4096

// x = embed ? dequant(token row) : X (+ TMP if add); X = x when it changed;
// y = (x * (1/sqrt(mean(x^2) + eps))) * gamma; y quantized per 32 into xq/xs.
// One workgroup; element i = j*256 + t so every 32-block sits in half a wave.
__global__ __launch_bounds__(NQ_WG) void k_resnorm_quant(NormQuantArgs a) {
    __shared__ double red_d[NQ_WG / 64];
    const int t = threadIdx.x, D = a.dim;
    const int per = D / NQ_WG;
    float xv[NQ_MAX_PER_THREAD];
    double ss = 0.0;
    const uint32_t tok = a.embed_qs ? *a.token : 0u;
#pragma unroll
    for (int j = 0; j < NQ_MAX_PER_THREAD; j++) {
        if (j < per) {
            const int i = j * NQ_WG + t;
            float v;
            if (a.embed_qs) {
                const int64_t row = (int64_t)tok;
                v = uq_half(a.embed_d[row * (D / 32) + i / 32]) * (float)a.embed_qs[row * D + i];
                a.x[i] = v;
            } else {
                v = a.x[i];
                if (a.add) {
                    v = v + a.residual[i];
                    a.x[i] = v;
                }
            }
            xv[j] = v;
            const float sq = v * v;
            ss += (double)sq;
        }
    }
    ss = block_sum_d<NQ_WG>(ss, red_d);
    const float mean = (float)(ss / (double)D);
    const float scale = 1.0f / sqrtf(mean + a.eps);
#pragma unroll
    for (int j = 0; j < NQ_MAX_PER_THREAD; j++) {
        if (j < per) {
            const int i = j * NQ_WG + t;
            const float tmp = xv[j] * scale;
            const float y = tmp * a.gamma[i];
            if (a.y) a.y[i] = y;
            float s;
            const int8_t q = uq_quant_lane(y, &s);
            a.xq[i] = q;
            if ((t & 31) == 0) a.xs[i >> 5] = s;
        }
    }
}

// q/k bias + NeoX rotate-half RoPE from the shared table, v bias; k and v are
// rounded to fp16 and stored at the current position of this layer's cache.
__global__ __launch_bounds__(256) void k_rope_kv(RopeArgs a) {
    const int pos = *a.pos;
    const int hd = a.head_dim, half = hd / 2;
    const float* trig = a.trig + (size_t)pos * hd;
    const int qpairs = a.heads * half, kpairs = a.kv_heads * half, kvd = a.kv_heads * hd;
    float* q = a.qkv;
    float* k = a.qkv + a.heads * hd;
    const float* v = k + kvd;
    uint16_t* kc = a.kcache + (size_t)pos * kvd;
    uint16_t* vc = a.vcache + (size_t)pos * kvd;
    for (int i = threadIdx.x; i < qpairs + kpairs + kvd; i += blockDim.x) {
        if (i < qpairs + kpairs) {
            const bool isq = i < qpairs;
            const int p = isq ? i : i - qpairs;
            const int h = p / half, j = p % half, ia = h * hd + j, ib = ia + half;
            float* base = isq ? q : k;
            const float* bias = isq ? a.bq : a.bk;
            const float cs = trig[j], sn = trig[half + j];
            const float u = bias ? base[ia] + bias[ia] : base[ia];
            const float w = bias ? base[ib] + bias[ib] : base[ib];
            const float p0 = u * cs, p1 = w * sn, p2 = u * sn, p3 = w * cs;
            const float ra = p0 - p1, rb = p2 + p3;
            if (isq) {
                base[ia] = ra;
                base[ib] = rb;
            } else {
                kc[ia] = uq_f16_rne(ra);
                kc[ib] = uq_f16_rne(rb);
            }
        } else {
            const int e = i - qpairs - kpairs;
            const float vb = a.bv ? v[e] + a.bv[e] : v[e];
            vc[e] = uq_f16_rne(vb);
        }
    }
}

// GQA attention for one query head per workgroup (1024 threads):
// s_t = (q . k_t) * (1/sqrt(hd)) with the dot summed in double; softmax with
// max subtraction, exp, total summed in double, p_t = e_t / total;
// out = sum_t p_t v_t in double (8 partials per dim, combined in LDS);
// the head's output is quantized per 32 in place (quant_act of gpu_graph.rs:148).
constexpr int AT_WG = 1024;
__global__ __launch_bounds__(AT_WG) void k_attention(AttnArgs a) {
    extern __shared__ float sc[];  // [max_seq] scores, then partials
    __shared__ double red_d[AT_WG / 64];
    __shared__ float red_f[AT_WG / 64];
    const int pos = *a.pos, T = pos + 1;
    const int h = blockIdx.x, hd = a.head_dim, kvd = a.kv_heads * hd;
    const int kh = h / (a.heads / a.kv_heads);
    const float* q = a.q + h * hd;
    const float qscale = a.qscale;
    float mx = -3.402823466e38f;
    for (int t = threadIdx.x; t < T; t += AT_WG) {
        const uint16_t* kr = a.kcache + (size_t)t * kvd + kh * hd;
        double acc = 0.0;
        for (int d = 0; d < hd; d += 8) {
            const int4 kk = *(const int4*)(kr + d);
            const uint32_t w[4] = {(uint32_t)kk.x, (uint32_t)kk.y, (uint32_t)kk.z, (uint32_t)kk.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                acc = __builtin_fma((double)q[d + 2 * e], (double)uq_half((uint16_t)(w[e] & 0xffff)), acc);
                acc = __builtin_fma((double)q[d + 2 * e + 1], (double)uq_half((uint16_t)(w[e] >> 16)), acc);
            }
        }
        const float s = (float)acc * qscale;
        sc[t] = s;
        mx = fmaxf(mx, s);
    }
    mx = block_max_f<AT_WG>(mx, red_f);
    double tot = 0.0;
    for (int t = threadIdx.x; t < T; t += AT_WG) {
        const float e = uq_expf(sc[t] - mx);
        sc[t] = e;
        tot += (double)e;
    }
    tot = block_sum_d<AT_WG>(tot, red_d);  // includes the barrier that publishes sc[]
    const float total = (float)tot;
    for (int t = threadIdx.x; t < T; t += AT_WG) sc[t] = sc[t] / total;
    __syncthreads();
    // P.V: thread = (dim d, slice r of 8); sequential over its t, then LDS sum
    const int d = threadIdx.x % hd, r = threadIdx.x / hd, R = AT_WG / hd;
    double acc = 0.0;
    for (int t = r; t < T; t += R)
        acc = __builtin_fma((double)sc[t], (double)uq_half(a.vcache[(size_t)t * kvd + kh * hd + d]), acc);
    double* part = (double*)(sc + ((a.max_seq + 1) & ~1));
    part[r * hd + d] = acc;
    __syncthreads();
    if (threadIdx.x < hd) {
        double s = 0.0;
        for (int rr = 0; rr < R; rr++) s += part[rr * hd + threadIdx.x];
        const float o = (float)s;
        a.out[h * hd + threadIdx.x] = o;
        float qs;
        const int8_t qv = uq_quant_lane(o, &qs);  // hd is a multiple of 32: blocks stay in one head
        a.xq[h * hd + threadIdx.x] = qv;
        if ((threadIdx.x & 31) == 0) a.xs[(h * hd + threadIdx.x) >> 5] = qs;
    }
}

// Greedy (stable argmax: lowest id wins ties; any non-finite logit marks the
// result bad). Each workgroup scans 2048 logits; the last workgroup to finish
// (atomic ticket, reset by that workgroup) reduces the partials, publishes the
// token for the next step, appends it to the history and advances the position.
struct Cand {
    float v;
    int id;
    unsigned bad;
    unsigned pad;
};
__device__ __forceinline__ bool better(float a, int ai, float b, int bi) { return a > b || (a == b && ai < bi); }
__device__ void cand_reduce(float& v, int& id, unsigned& bad, float* vs, int* ids, unsigned* bs) {
    const int t = threadIdx.x;
    vs[t] = v;
    ids[t] = id;
    bs[t] = bad;
    __syncthreads();
    for (int d = blockDim.x / 2; d; d >>= 1) {
        if (t < d) {
            if (better(vs[t + d], ids[t + d], vs[t], ids[t])) {
                vs[t] = vs[t + d];
                ids[t] = ids[t + d];
            }
            bs[t] |= bs[t + d];
        }
        __syncthreads();
    }
    v = vs[0];
    id = ids[0];
    bad = bs[0];
}
constexpr int GR_WG = 256, GR_TILE = 2048;
__global__ __launch_bounds__(GR_WG) void k_greedy(GreedyArgs a) {
    __shared__ float vs[GR_WG];
    __shared__ int ids[GR_WG];
    __shared__ unsigned bs[GR_WG];
    __shared__ bool last;
    float best = -__builtin_inff();
    int id = 0x7fffffff;
    unsigned bad = 0;
    for (int j = 0; j < GR_TILE / GR_WG; j++) {
        const int i = blockIdx.x * GR_TILE + j * GR_WG + threadIdx.x;
        if (i < a.n) {
            const float v = a.logits[i];
            bad |= (__float_as_uint(v) & 0x7f800000u) == 0x7f800000u;
            if (better(v, i, best, id)) {
                best = v;
                id = i;
            }
        }
    }
    cand_reduce(best, id, bad, vs, ids, bs);
    Cand* part = (Cand*)a.partial;
    if (threadIdx.x == 0) {
        part[blockIdx.x] = Cand{best, id, bad, 0u};
        __threadfence();
        const unsigned ticket = atomicAdd(a.ticket, 1u);
        last = ticket == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    best = -__builtin_inff();
    id = 0x7fffffff;
    bad = 0;
    for (int j = threadIdx.x; j < (int)gridDim.x; j += GR_WG) {
        const volatile Cand* c = (const volatile Cand*)part + j;
        const float cv = c->v;
        const int cid = c->id;
        bad |= c->bad;
        if (better(cv, cid, best, id)) {
            best = cv;
            id = cid;
        }
    }
    cand_reduce(best, id, bad, vs, ids, bs);
    if (threadIdx.x == 0) {
        *a.ticket = 0u;
        a.result[0] = (uint32_t)id;
        a.result[1] = bad;
        if (a.token) {
            const int pos = *a.pos;
            *a.token = (uint32_t)id;
            if (a.history && pos < a.max_seq) a.history[pos] = (uint32_t)id;
            *a.pos = pos + 1;
        }
    }
}

}  // namespace

void launch_resnorm_quant(const NormQuantArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_resnorm_quant, dim3(1), dim3(NQ_WG), 0, s, a);
}
void launch_rope_kv(const RopeArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_rope_kv, dim3(1), dim3(256), 0, s, a);
}
void launch_attention(const AttnArgs& a, hipStream_t s) {
    const size_t lds = sizeof(float) * (size_t)((a.max_seq + 1) & ~1) + sizeof(double) * AT_WG;
    hipLaunchKernelGGL(k_attention, dim3(a.heads), dim3(AT_WG), lds, s, a);
}
void launch_greedy(const GreedyArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_greedy, dim3((a.n + GR_TILE - 1) / GR_TILE), dim3(GR_WG), 0, s, a);
}
int greedy_partials(int n) { return (n + GR_TILE - 1) / GR_TILE; }

}  // namespace uq
