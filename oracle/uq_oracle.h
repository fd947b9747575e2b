/*
 * CPU oracle for the quantized-matmul hot path (TEST INFRASTRUCTURE ONLY).
 *
 * A single-file C restatement of the reference runtime's arithmetic, written
 * from the Rust/CUDA text of nodnarbrox/uefi-gpu. Only tests/, the smoke check
 * and the CPU-baseline leg of bench.py may load it; the product library never
 * links, calls or falls back to it.
 *
 * Every function names the reference file:line it restates. Shared numeric
 * conventions (apply to the oracle and to the HIP kernels alike):
 *   - elementwise f32 arithmetic is written op by op and built with
 *     -ffp-contract=off (driver/kernels/compile_ops.py:9 compiles --fmad=false);
 *   - every reduction (dot sums, RMSNorm sum of squares, softmax denominators,
 *     attention P.V) accumulates exactly-formed terms in double and rounds to f32
 *     once, the form of driver/src/frontier_forward.rs:38-42; the result is then
 *     independent of summation order up to ~2^-29 relative, so the GPU may sum
 *     in any order and still agree bit for bit (see uqo_* docstrings);
 *   - the Q8_0 prefill GEMM keeps the reference's sequential per-32-block f32
 *     fmaf update (driver/kernels/gpu_prefill.cu:29-30), mirrored exactly;
 *   - exp is uqo_expf, the libm 0.2.16 expf of the reference's Rust path
 *     (FreeBSD e_expf.c; driver/src/frontier_cpu_expf.rs:80-170), in f32.
 *
 * Parity status per function is listed in the header of uq_oracle.c.
 */
#ifndef UQ_ORACLE_H
#define UQ_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF quant kinds used on this path (ggml type ids). */
enum { UQO_F32 = 0, UQO_Q8_0 = 8, UQO_Q3_K = 11, UQO_Q4_K = 12, UQO_Q6_K = 14, UQO_IQ3_XXS = 18,
       UQO_IQ4_NL = 20, UQO_IQ4_XS = 23, UQO_BF16 = 30 };

void     uqo_set_threads(int n);
int      uqo_get_threads(void);

float    uqo_half(uint16_t h);
uint16_t uqo_f16_rne(float f);
float    uqo_expf(float x);
int64_t  uqo_row_bytes(uint32_t kind, int64_t n);
int      uqo_dequantize(uint32_t kind, const uint8_t* in, int64_t n, float* out);
uint32_t uqo_iq3_grid(int i);
int      uqo_iq4_value(int i);
void     uqo_linear(uint32_t kind, const uint8_t* w, int64_t n, int64_t m, const float* x, float* y);
void     uqo_linear_f32seq(uint32_t kind, const uint8_t* w, int64_t n, int64_t m, const float* x, float* y);
int64_t  uqo_frontier_fixture(uint32_t kind, int64_t n, uint8_t* out);

void uqo_quant_act(const float* x, int64_t n, float* scale, int8_t* q);

void uqo_q8_block_dots(const uint8_t* w, int64_t n, int64_t m, const int8_t* qx, int32_t* dots);
void uqo_q4k_block_dots(const uint8_t* w, int64_t n, int64_t m, const int8_t* qx, int32_t* dots);
void uqo_q3k_block_dots(const uint8_t* w, int64_t n, int64_t m, const int8_t* qx, int32_t* dots);
void uqo_matvec(uint32_t kind, const uint8_t* w, int64_t n, int64_t m,
                const float* xscale, const int8_t* qx, float* y);
void uqo_matvec_x(uint32_t kind, const uint8_t* w, int64_t n, int64_t m, const float* x, float* y);
void uqo_q8_matvec_f32seq(const uint8_t* w, int64_t n, int64_t m, const float* x, float* y);
void uqo_q8_dequant_dot(const uint8_t* w, int64_t n, int64_t m, const float* x, float* y);

void uqo_prefill_gemm(const uint8_t* w, int64_t n, int64_t m, int64_t batch,
                      const float* xscale, const int8_t* qx, float* y);

void uqo_rmsnorm(const float* x, const float* gamma, int64_t n, float eps, float* y);
void uqo_rope_table(int seq, int head_dim, float theta, float* table);
void uqo_rope_bias(float* v, const float* bias, int heads, int head_dim, const float* trig_row);
float uqo_silu_mul(float g, float u);
void uqo_attention(const float* q, const uint16_t* keys, const uint16_t* values, int pos,
                   int heads, int kv_heads, int head_dim, float* out);
int  uqo_greedy(const float* logits, int64_t n, int* bad);

/* Qwen2 dense decoder (driver/src/llm.rs:313-388, gpu_graph.rs:137-162,
 * gpu_prefill.rs:122-150). Tensors are GGUF-layout bytes. */
typedef struct {
    const float   *attn_norm, *ffn_norm, *bq, *bk, *bv;
    const uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd; /* Q8_0 */
} uqo_layer;

typedef struct {
    int32_t layers, dim, hidden, heads, kv_heads, head_dim, vocab, max_seq;
    float   eps, theta;
    const uint8_t  *tok_embd;    /* Q8_0 vocab x dim */
    const float    *output_norm; /* dim */
    const uint8_t  *output;      /* Q8_0 vocab x dim */
    const uqo_layer* layer;      /* [layers] */
} uqo_qwen2;

typedef struct uqo_state uqo_state;
uqo_state* uqo_state_new(const uqo_qwen2* m);
void       uqo_state_free(uqo_state* s);
int  uqo_prefill(uqo_state* s, const uint32_t* tokens, int count, uint32_t* next, float* logits);
int  uqo_decode(uqo_state* s, uint32_t token, int pos, uint32_t* next, float* logits);
const uint16_t* uqo_state_keys(const uqo_state* s, int layer);
const uint16_t* uqo_state_values(const uqo_state* s, int layer);

/* Reference-order decode (gpu_graph.rs:137-162 kernels' f32 orders; see the
 * section comment in uq_oracle.c). kv_fp16: round cached K/V to fp16. */
typedef struct uqo_refo uqo_refo;
uqo_refo* uqo_refo_new(const uqo_qwen2* m, int kv_fp16);
void      uqo_refo_free(uqo_refo* s);
int  uqo_refo_decode(uqo_refo* s, uint32_t token, int pos, uint32_t* next, float* logits);
void uqo_refo_resnorm(float* x, const float* residual, const float* w, float* y, int n, float eps, int add);
float uqo_refo_dotrow(const uint8_t* w, const float* xs, const int8_t* xq, int64_t blocks);
float uqo_refo_linear_row(const uint8_t* w, const float* xs, const int8_t* xq, int64_t blocks);
void uqo_refo_attention_head(const float* q, const float* keys, const float* values, int pos, int kvd, int kh,
                             int hd, float* out);

/* MoE expert FFN (driver/src/frontier_forward.rs:164-199). */
typedef struct {
    int32_t dim, ff, experts, top_k;
    uint32_t expert_kind;          /* UQO_Q3_K (config) or any supported kind */
    const uint8_t* const* gate;    /* [experts] ff x dim   */
    const uint8_t* const* up;      /* [experts] ff x dim   */
    const uint8_t* const* down;    /* [experts] dim x ff   */
    uint32_t shared_kind;          /* UQO_Q8_0 */
    const uint8_t *sh_gate, *sh_up, *sh_down;
    const float   *sh_scale;       /* dim, f32: ffn_gate_inp_shexp (NULL: weight 1) */
} uqo_moe;

int uqo_moe_route(const float* logits, int experts, int top_k, int32_t* ids, float* weights);
int uqo_moe_ffn(const uqo_moe* moe, const float* x, const float* router_logits, float* out,
                int32_t* ids_out, float* weights_out);

#ifdef __cplusplus
}
#endif
#endif
