// Argument blocks and launchers of the fused decode-step kernels (uq_step.hip).
// All matrices are Q8_0 planes (int8 quants [rows][k], fp16 scales [rows][k/32]).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "uq_decode.h"

namespace uq {

constexpr int LM_MAX_WG = 2048;  // lm_head grid cap == argmax partial slots

struct QkvArgs {
    const int8_t* w_qs;       // [heads*hd + 2*kv*hd][dim]
    const uint16_t* w_d;
    NormQuantArgs nq;         // prologue: residual sum, RMSNorm, quant of the input
    const float *bq, *bk, *bv;
    const float* trig;        // [max_seq][hd]
    const int* pos;
    float* q;                 // rotated q [heads*hd]
    uint16_t* kcache;         // this layer [max_seq][kv*hd]
    uint16_t* vcache;
    int dim, heads, kv_heads, head_dim;
};

// Gate/up of the decode FFN: h = silu(gate x) * (up x) in f32, with the
// residual + RMSNorm + quant of the input in the prologue. One workgroup per
// CU, rows split evenly over the grid.
struct GateArgs {
    const int8_t *g_qs, *u_qs;
    const uint16_t *g_d, *u_d;
    NormQuantArgs nq;         // prologue: residual sum, RMSNorm, quant of the input
    float* h;                 // silu(g)*u [rows]
    int64_t rows, k;
    int64_t share;            // rows / grid, set by the launcher
};

// Down projection y = W quant(h): the block-32 quant of h happens in the
// kernel's prologue, in the waves that have no rows to stream.
struct DownArgs {
    const int8_t* w_qs;
    const uint16_t* w_d;
    const float* h;           // [k]
    float* y;                 // [rows]
    int64_t rows, k;
    int64_t share;            // rows / grid, set by the launcher
};

struct LmArgs {
    const int8_t* w_qs;
    const uint16_t* w_d;
    const int8_t* xq;
    const float* xs;
    float* logits;
    int64_t rows, k;
    void* partial;            // [LM_MAX_WG] 16-byte candidates
    uint32_t* result;         // [0] id, [1] bad, [2] sticky bad
    uint32_t* token;          // optional next-step token feedback
    int* pos;
    uint32_t* history;
    int max_seq;
    NormQuantArgs nq;         // the output RMSNorm + quant of the input, done by every workgroup
};

// Decode attention split over ATT_SPLIT position chunks per query head:
// scores -> [heads][max_seq] and per-chunk maxima, then each chunk's P.V
// (with the exact global softmax) added into a double accumulator, which the
// o projection reads, converts and quantizes in its prologue. 16 chunks
// (192 workgroups for 12 heads) measured fastest at positions 512..640 of the
// Qwen2.5-1.5B shape: 1011-1015 tok/s against 983 with 8, 943 with 4, 990
// with 24 and 998 with 32.
constexpr int ATT_SPLIT = 16;
struct AttSplitArgs {
    const float* q;           // rotated q [heads*hd]
    const uint16_t* kcache;   // this layer [max_seq][kv*hd]
    const uint16_t* vcache;
    const int* pos;
    float* scores;            // [heads][max_seq]
    float* cmax;              // [heads][ATT_SPLIT]
    double* acc;              // [heads*hd], zeroed by the scores kernel
    int heads, kv_heads, head_dim, max_seq;
    float qscale;
};

// o projection with the attention accumulator as input: y = W quant((float)acc)
struct WoArgs {
    const int8_t* w_qs;
    const uint16_t* w_d;
    const double* acc;        // [k]
    float* y;                 // [rows]
    int64_t rows, k;
    int64_t share;            // rows / grid, set by the launcher
};

int launch_qkv_rope(const QkvArgs& a, hipStream_t s);
int launch_attention_split(const AttSplitArgs& a, hipStream_t s);
int launch_wo_acc(const WoArgs& a, hipStream_t s);
int launch_gateup_h(const GateArgs& a, hipStream_t s);
int launch_down_h(const DownArgs& a, hipStream_t s);
int launch_lm_greedy(const LmArgs& a, hipStream_t s);

}  // namespace uq
