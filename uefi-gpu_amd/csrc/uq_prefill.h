// Argument blocks and launchers of the prefill kernels (uq_prefill.hip).
// Token-major activations: x[t][dim] f32, xq[t][k] int8, xst[k/32][mp] f32
// (scales transposed so a GEMM lane reads its token's scale with one load);
// mp = token count padded to the GEMM tile (64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "uq_decode.h"

namespace uq {

struct PfNormArgs {
    NormQuantArgs nq;        // gamma, eps, dim, embedding planes (layer 0)
    float* x;                // residual rows [n][dim], updated in place
    const float* residual;   // added rows [n][dim] (null for the embedding)
    const uint32_t* tokens;  // token ids [n] when embedding
    int8_t* xq;              // [mp][dim]
    float* xst;              // [dim/32][mp]
    int mp;
};

// The q|k|v GEMM's bias + RoPE + KV epilogue (prefill_rope, gpu_prefill.cu:
// 73-81, fused into the GEMM): the weight's rows are permuted so that within
// every q and k head row 2j + e holds the head's output j + e * head_dim/2
// (the RoPE partners adjacent: a lane's 4 consecutive rows are two pairs);
// v rows keep their order. The bias is permuted likewise (a region without a
// bias adds nothing). q is written rotated to q[t][...] in the original order,
// k and v rounded to fp16 into the caches at position p0 + t, for t < n.
struct PfRopeEpi {
    float* q;                // rows [mp][stride]; their q part is written
    int stride;
    const float* bias;       // permuted q|k|v bias (one float per row)
    int hb_q, hb_k, hb_v;    // which regions have a bias
    const float* trig;       // RoPE table [position][head_dim]: cos | sin
    uint16_t* kcache;        // this layer
    uint16_t* vcache;
    int n, p0, heads, kv_heads, head_dim;
};

struct PfGemmArgs {
    const int8_t* w_qs;      // [n][k]
    const float* w_ds;       // weight scales widened to f32, transposed [k/32][n]
    const int8_t* w2_qs;     // second matrix (up) for the gate/up SiLU epilogue, or null
    const float* w2_ds;
    const int8_t* xq;        // [mp][k]
    const float* xst;        // [k/32][mp]
    float* y;                // [mp][n]
    int64_t n, k;
    int mp;
    // gate/up only, instead of y: SiLU(gate)*up quantized per 32 rows, codes
    // [mp][n] and scales [n/32][mp] (the next GEMM's input planes), or null
    int8_t* yq;
    float* yst;
    // the q|k|v launch only (rows permuted as PfRopeEpi says), instead of y
    int rope;
    PfRopeEpi re;
};

struct PfAttnArgs {
    const float* qkv;        // rotated q rows [n][stride]
    int stride;
    const uint16_t* kcache;
    const uint16_t* vcache;
    float* out;              // [n][heads*hd]
    int n, p0, kcap;         // queries, first position, positions allocated in the caches (>= p0 + n)
    int heads, kv_heads, head_dim;
    float qscale;
    // head_dim 128 only, instead of out: the output quantized per 32 dims
    // (codes [n][heads*hd], scales [heads*hd/32][mp]: the o GEMM's input planes), or null
    int8_t* xq;
    float* xst;
    int mp;
    int ncu;                 // set by the launcher: the CU count (workgroup pairing order)
};

void launch_transpose_scales(const uint16_t* d, int64_t rows, int64_t nb, float* dt, hipStream_t s);
void launch_pf_norm(const PfNormArgs& a, int tokens, hipStream_t s);
void launch_pf_quant(const float* x, int64_t k, int tokens, int mp, int8_t* xq, float* xst, hipStream_t s);
int launch_pf_gemm(const PfGemmArgs& a, hipStream_t s);
// dst row r = src row perm[r] (rows of rowb bytes, rowb % 16 == 0), and the
// same gather on the columns of a [nb][m] float plane
void launch_gather_rows(const int8_t* src, int64_t rowb, const int* perm, int64_t m, int8_t* dst, hipStream_t s);
void launch_gather_cols(const float* src, int64_t nb, int64_t m, const int* perm, float* dst, hipStream_t s);
int launch_pf_attention(const PfAttnArgs& a, hipStream_t s);

}  // namespace uq
