// Argument blocks and launchers of the decode-step kernels (uq_decode.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace uq {

struct NormQuantArgs {
    float* x;                // residual stream [dim] (read, and written when it changes)
    const float* residual;   // added to x when add != 0
    const float* gamma;      // RMSNorm weight [dim]
    float* y;                // optional normalized output [dim]
    int8_t* xq;              // quantized normalized output [dim]
    float* xs;               // per-32 scales [dim/32]
    const int8_t* embed_qs;  // when set: x = dequant(token row) (Q8_0 planes)
    const uint16_t* embed_d;
    const uint32_t* token;
    int dim;
    int add;
    float eps;
};

struct RopeArgs {
    float* qkv;              // [heads*hd | kv*hd | kv*hd]
    const float *bq, *bk, *bv;
    const float* trig;       // [max_seq][hd]: cos | sin
    const int* pos;
    uint16_t* kcache;        // this layer, [max_seq][kv*hd] fp16
    uint16_t* vcache;
    int heads, kv_heads, head_dim;
};

struct AttnArgs {
    const float* q;
    const uint16_t* kcache;
    const uint16_t* vcache;
    const int* pos;
    float* out;              // [heads*hd]
    int8_t* xq;              // quantized out
    float* xs;
    int heads, kv_heads, head_dim, max_seq;
    float qscale;
};

struct GreedyArgs {
    const float* logits;
    int n;
    void* partial;           // [greedy_partials(n)] 16-byte candidates
    unsigned* ticket;        // zero between launches (the last workgroup resets it)
    uint32_t* result;        // [0] = id, [1] = bad
    uint32_t* token;         // optional: next-step token (decode feedback)
    int* pos;                // advanced when token is set
    uint32_t* history;       // optional: history[pos] = id
    int max_seq;
};

void launch_resnorm_quant(const NormQuantArgs& a, hipStream_t s);
void launch_rope_kv(const RopeArgs& a, hipStream_t s);
void launch_attention(const AttnArgs& a, hipStream_t s);
void launch_greedy(const GreedyArgs& a, hipStream_t s);
int greedy_partials(int n);

}  // namespace uq
