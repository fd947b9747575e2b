// Q8_0 prompt prefill for gfx950: int8 MFMA GEMM with the per-32-block
// rescale, and the batched norm / quant / RoPE / causal attention around it.
//
// Replaces prefill_gemm / prefill_repack / prefill_quant / prefill_resnorm /
// prefill_rope / prefill_attention / silu_mul (driver/kernels/gpu_prefill.cu:
// 74-165, gpu_ops.cu:266-268) and the stream built by prepare_prefill
// (driver/src/gpu_prefill.rs:122-150).
//
// GEMM: y[t][r] = sum over 32-blocks b, in order, of
//   f = fmaf((float)c_b, dw[r][b] * dx[t][b], f),   c_b = sum_k qw[r][k] qx[t][k]
// (gpu_prefill.cu:93-94). c_b is one v_mfma_i32_16x16x32_i8 per block with a
// zero accumulator; the f32 rescale runs on the VALU in the same order as the
// reference, so results match the oracle bit for bit.
// Operands come straight from the row-major planes used by decode (no second
// weight copy); only the fp16 weight scales get a [block][row] transpose so a
// lane reads its four rows' scales with one 8-byte load.
#include "uq_device.h"
#include "uq_blockops.h"
#include "uq_prefill.h"

namespace uq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ scale transpose
__global__ __launch_bounds__(256) void k_transpose_scales(const uint16_t* __restrict__ d, int64_t rows, int64_t nb,
                                                          uint16_t* __restrict__ dt) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * nb) return;
    const int64_t r = i / nb, b = i % nb;
    dt[b * rows + r] = d[i];
}

// ------------------------------------------------------------------ per-token norm + quant
// One workgroup per token: x = embed(token) or x + residual (stored back),
// RMSNorm, block-32 quant into xq[t][dim] and xsT[b][t].
__global__ __launch_bounds__(256) void k_pf_norm(PfNormArgs a) {
    __shared__ double red[4];
    const int t = blockIdx.x;
    NormQuantArgs nq = a.nq;
    nq.x = a.x + (size_t)t * a.nq.dim;
    nq.residual = a.residual ? a.residual + (size_t)t * a.nq.dim : nullptr;
    nq.x_out = a.x + (size_t)t * a.nq.dim;
    if (a.tokens) nq.token = a.tokens + t;
    norm_quant<256>(nq, true, a.xq + (size_t)t * a.nq.dim, a.xst + t, red, a.mp);
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
// Workgroup tile 64 rows x 64 tokens, four waves of 32 x 32 (2 x 2 MFMA tiles).
// MFMA 16x16x32 i8 lane layout: A lane l = row l%16, k (l/16)*8..+7; B lane l =
// token l%16, same k; D lane l = rows (l/16)*4..+3, token l%16.
template <bool GU>
__global__ __launch_bounds__(256) void k_pf_gemm(PfGemmArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * 64 + (wave >> 1) * 32;
    const int64_t t0 = (int64_t)blockIdx.y * 64 + (wave & 1) * 32;
    const int li = lane & 15, lk = (lane >> 4) * 8, lm = (lane >> 4) * 4;
    const int64_t K = a.k, N = a.n, nb = K / 32;
    const int8_t* A0 = a.w_qs + (r0 + li) * K + lk;
    const int8_t* A1 = A0 + 16 * K;
    const int8_t* G0 = GU ? a.w2_qs + (r0 + li) * K + lk : nullptr;
    const int8_t* G1 = GU ? G0 + 16 * K : nullptr;
    const int8_t* B0 = a.xq + (t0 + li) * K + lk;
    const int8_t* B1 = B0 + 16 * K;
    float f[2][2][4], g[2][2][4];
#pragma unroll
    for (int x = 0; x < 2; x++)
#pragma unroll
        for (int y = 0; y < 2; y++)
#pragma unroll
            for (int m = 0; m < 4; m++) f[x][y][m] = g[x][y][m] = 0.0f;
    const v4i z = {0, 0, 0, 0};
    for (int64_t b = 0; b < nb; b++) {
        const long a0 = *(const long*)(A0 + 32 * b), a1 = *(const long*)(A1 + 32 * b);
        const long b0 = *(const long*)(B0 + 32 * b), b1 = *(const long*)(B1 + 32 * b);
        const uint2 d0 = *(const uint2*)(a.w_dt + b * N + r0 + lm);
        const uint2 d1 = *(const uint2*)(a.w_dt + b * N + r0 + 16 + lm);
        const float x0 = a.xst[b * a.mp + t0 + li], x1 = a.xst[b * a.mp + t0 + 16 + li];
        const v4i c00 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, b0, z, 0, 0, 0);
        const v4i c01 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, b1, z, 0, 0, 0);
        const v4i c10 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, b0, z, 0, 0, 0);
        const v4i c11 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, b1, z, 0, 0, 0);
        const float w0[4] = {uq_half((uint16_t)(d0.x & 0xffff)), uq_half((uint16_t)(d0.x >> 16)),
                             uq_half((uint16_t)(d0.y & 0xffff)), uq_half((uint16_t)(d0.y >> 16))};
        const float w1[4] = {uq_half((uint16_t)(d1.x & 0xffff)), uq_half((uint16_t)(d1.x >> 16)),
                             uq_half((uint16_t)(d1.y & 0xffff)), uq_half((uint16_t)(d1.y >> 16))};
#pragma unroll
        for (int m = 0; m < 4; m++) {
            f[0][0][m] = fmaf((float)c00[m], w0[m] * x0, f[0][0][m]);
            f[0][1][m] = fmaf((float)c01[m], w0[m] * x1, f[0][1][m]);
            f[1][0][m] = fmaf((float)c10[m], w1[m] * x0, f[1][0][m]);
            f[1][1][m] = fmaf((float)c11[m], w1[m] * x1, f[1][1][m]);
        }
        if (GU) {
            const long g0 = *(const long*)(G0 + 32 * b), g1 = *(const long*)(G1 + 32 * b);
            const uint2 e0 = *(const uint2*)(a.w2_dt + b * N + r0 + lm);
            const uint2 e1 = *(const uint2*)(a.w2_dt + b * N + r0 + 16 + lm);
            const v4i h00 = __builtin_amdgcn_mfma_i32_16x16x32_i8(g0, b0, z, 0, 0, 0);
            const v4i h01 = __builtin_amdgcn_mfma_i32_16x16x32_i8(g0, b1, z, 0, 0, 0);
            const v4i h10 = __builtin_amdgcn_mfma_i32_16x16x32_i8(g1, b0, z, 0, 0, 0);
            const v4i h11 = __builtin_amdgcn_mfma_i32_16x16x32_i8(g1, b1, z, 0, 0, 0);
            const float u0[4] = {uq_half((uint16_t)(e0.x & 0xffff)), uq_half((uint16_t)(e0.x >> 16)),
                                 uq_half((uint16_t)(e0.y & 0xffff)), uq_half((uint16_t)(e0.y >> 16))};
            const float u1[4] = {uq_half((uint16_t)(e1.x & 0xffff)), uq_half((uint16_t)(e1.x >> 16)),
                                 uq_half((uint16_t)(e1.y & 0xffff)), uq_half((uint16_t)(e1.y >> 16))};
#pragma unroll
            for (int m = 0; m < 4; m++) {
                g[0][0][m] = fmaf((float)h00[m], u0[m] * x0, g[0][0][m]);
                g[0][1][m] = fmaf((float)h01[m], u0[m] * x1, g[0][1][m]);
                g[1][0][m] = fmaf((float)h10[m], u1[m] * x0, g[1][0][m]);
                g[1][1][m] = fmaf((float)h11[m], u1[m] * x1, g[1][1][m]);
            }
        }
    }
#pragma unroll
    for (int x = 0; x < 2; x++)
#pragma unroll
        for (int y = 0; y < 2; y++) {
            const int64_t t = t0 + 16 * y + li, r = r0 + 16 * x + lm;
            float4 o;
            if (GU) {
                o = make_float4(uq_silu_mul(f[x][y][0], g[x][y][0]), uq_silu_mul(f[x][y][1], g[x][y][1]),
                                uq_silu_mul(f[x][y][2], g[x][y][2]), uq_silu_mul(f[x][y][3], g[x][y][3]));
            } else {
                o = make_float4(f[x][y][0], f[x][y][1], f[x][y][2], f[x][y][3]);
            }
            *(float4*)(a.y + t * N + r) = o;
        }
}

// ------------------------------------------------------------------ RoPE + KV
// One workgroup per token: q/k bias + RoPE (q in place), k and v rounded to
// fp16 into the cache at position p0 + t (prefill_rope, gpu_prefill.cu:137-145).
__global__ __launch_bounds__(256) void k_pf_rope_kv(PfRopeArgs a) {
    const int t = blockIdx.x, pos = a.p0 + t;
    const int hd = a.head_dim, half = hd / 2, kvd = a.kv_heads * hd;
    const int qpairs = a.heads * half, kpairs = a.kv_heads * half;
    float* row = a.qkv + (size_t)t * a.stride;
    float* q = row;
    const float* k = row + a.heads * hd;
    const float* v = k + kvd;
    const float* trig = a.trig + (size_t)pos * hd;
    uint16_t* kc = a.kcache + (size_t)pos * kvd;
    uint16_t* vc = a.vcache + (size_t)pos * kvd;
    for (int i = threadIdx.x; i < qpairs + kpairs + kvd; i += 256) {
        if (i < qpairs + kpairs) {
            const bool isq = i < qpairs;
            const int p = isq ? i : i - qpairs;
            const int h = p / half, j = p % half, ia = h * hd + j, ib = ia + half;
            const float* base = isq ? q : k;
            const float* bias = isq ? a.bq : a.bk;
            const float cs = trig[j], sn = trig[half + j];
            const float u = bias ? base[ia] + bias[ia] : base[ia];
            const float w = bias ? base[ib] + bias[ib] : base[ib];
            const float p0 = u * cs, p1 = w * sn, p2 = u * sn, p3 = w * cs;
            const float ra = p0 - p1, rb = p2 + p3;
            if (isq) {
                q[ia] = ra;
                q[ib] = rb;
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

// ------------------------------------------------------------------ causal attention
// Workgroup = (query head, tile of QT consecutive queries); 32 threads per query.
// Same arithmetic as decode attention: scores in double, * 1/sqrt(hd),
// max-subtracted exp, total in double, p = e/total, P.V in double.
constexpr int QT = 8;
template <int HD>
__global__ __launch_bounds__(256) void k_pf_attention(PfAttnArgs a) {
    extern __shared__ float scs[];  // [QT][kmax]
    __shared__ double qd[QT][HD];
    const int tid = threadIdx.x, qi = tid >> 5, kj = tid & 31;
    const int h = blockIdx.x, kh = h / (a.heads / a.kv_heads), kvd = a.kv_heads * HD;
    const int tq0 = blockIdx.y * QT;                 // first query (token index)
    const int kmax = a.p0 + tq0 + QT;                // keys covered by this tile (exclusive bound)
    for (int e = tid; e < QT * HD; e += 256) {
        const int qq = e / HD, d = e % HD;
        const int t = tq0 + qq;
        qd[qq][d] = t < a.n ? (double)a.qkv[(size_t)t * a.stride + h * HD + d] : 0.0;
    }
    __syncthreads();
    const int tq = tq0 + qi;
    const bool live = tq < a.n;
    const int T = a.p0 + tq + 1;                     // causal: keys [0, T)
    float* sc = scs + qi * a.kcap;
    float mx = -3.402823466e38f;
    if (live) {
        for (int t = kj; t < T; t += 32) {
            const uint16_t* kr = a.kcache + (size_t)t * kvd + kh * HD;
            double acc = 0.0;
            for (int d = 0; d < HD; d += 8) {
                const int4 kk = *(const int4*)(kr + d);
                const uint32_t w[4] = {(uint32_t)kk.x, (uint32_t)kk.y, (uint32_t)kk.z, (uint32_t)kk.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    acc = __builtin_fma(qd[qi][d + 2 * i], (double)uq_half((uint16_t)(w[i] & 0xffff)), acc);
                    acc = __builtin_fma(qd[qi][d + 2 * i + 1], (double)uq_half((uint16_t)(w[i] >> 16)), acc);
                }
            }
            const float s = (float)acc * a.qscale;
            sc[t] = s;
            mx = fmaxf(mx, s);
        }
    }
    mx = uq_group_max<32>(mx);
    double tot = 0.0;
    if (live)
        for (int t = kj; t < T; t += 32) {
            const float ev = uq_expf(sc[t] - mx);
            sc[t] = ev;
            tot += (double)ev;
        }
    tot = uq_group_sum<32>(tot);
    const float total = (float)tot;
    if (live)
        for (int t = kj; t < T; t += 32) sc[t] = sc[t] / total;
    __syncthreads();  // p of every key visible to the 32 threads of the query
    (void)kmax;
    if (!live) return;
    // P.V: thread kj owns dims [kj*HD/32, +HD/32)
    constexpr int DPT = HD / 32;
    double acc[DPT];
#pragma unroll
    for (int i = 0; i < DPT; i++) acc[i] = 0.0;
    const uint16_t* vb = a.vcache + kh * HD + kj * DPT;
    for (int t = 0; t < T; t++) {
        const double p = (double)sc[t];
#pragma unroll
        for (int i = 0; i < DPT; i++) acc[i] = __builtin_fma(p, (double)uq_half(vb[(size_t)t * kvd + i]), acc[i]);
    }
    float* out = a.out + (size_t)tq * (a.heads * HD) + h * HD + kj * DPT;
#pragma unroll
    for (int i = 0; i < DPT; i++) out[i] = (float)acc[i];
}

}  // namespace

void launch_transpose_scales(const uint16_t* d, int64_t rows, int64_t nb, uint16_t* dt, hipStream_t s) {
    hipLaunchKernelGGL(k_transpose_scales, dim3((unsigned)((rows * nb + 255) / 256)), dim3(256), 0, s, d, rows, nb, dt);
}
void launch_pf_norm(const PfNormArgs& a, int tokens, hipStream_t s) {
    hipLaunchKernelGGL(k_pf_norm, dim3(tokens), dim3(256), 0, s, a);
}
void launch_pf_quant(const float* x, int64_t k, int tokens, int mp, int8_t* xq, float* xst, hipStream_t s) {
    hipLaunchKernelGGL(k_pf_quant, dim3((unsigned)((k + 255) / 256), tokens), dim3(256), 0, s, x, k, mp, xq, xst);
}
int launch_pf_gemm(const PfGemmArgs& a, hipStream_t s) {
    if (a.n % 64 || a.mp % 64 || a.k % 32) return -1;
    const dim3 grid((unsigned)(a.n / 64), (unsigned)(a.mp / 64));
    if (a.w2_qs) hipLaunchKernelGGL(k_pf_gemm<true>, grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(k_pf_gemm<false>, grid, dim3(256), 0, s, a);
    return 0;
}
void launch_pf_rope_kv(const PfRopeArgs& a, int tokens, hipStream_t s) {
    hipLaunchKernelGGL(k_pf_rope_kv, dim3(tokens), dim3(256), 0, s, a);
}
int launch_pf_attention(const PfAttnArgs& a, hipStream_t s) {
    const size_t lds = sizeof(float) * QT * (size_t)a.kcap;
    if (lds + sizeof(double) * QT * a.head_dim > 65536) return -1;
    const dim3 grid(a.heads, (a.n + QT - 1) / QT);
    switch (a.head_dim) {
    case 64: hipLaunchKernelGGL(k_pf_attention<64>, grid, dim3(256), lds, s, a); return 0;
    case 128: hipLaunchKernelGGL(k_pf_attention<128>, grid, dim3(256), lds, s, a); return 0;
    default: return -1;
    }
}

}  // namespace uq
