/*
 * uq -- C ABI of the MI355X (gfx950) quantized-matmul hot path.
 *
 * Drop-in for the call surface of the reference runtime nodnarbrox/uefi-gpu
 * (Rust, no_std UEFI). Each entry point names the reference interface it
 * replaces (file:line in that repository). Plain pointers and sizes only.
 *
 * Conventions (driver/src/llm.rs:110-273, frontier_forward.rs:10-28):
 *  - every call returns an int status: UQ_OK (0) or a negative UQ_ERR_*;
 *    uq_last_error() gives the message of the calling thread's last failure;
 *  - host-pointer calls are synchronous (the reference polls each submission
 *    to completion); *_dev calls take device pointers and enqueue on the
 *    library stream (or the given hipStream_t) without synchronizing;
 *  - one process context per GPU, single caller thread, no re-entrancy
 *    (the reference's `Gpu` object is used the same way);
 *  - weights are device resident after a verified upload (llm.rs:157-201).
 */
#ifndef UQ_H
#define UQ_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. frontier_forward.rs:10 Error {Backend, Shape, NonFinite, Context},
 * frontier_core.rs:37 Error::QuantType, llm.rs:267-269 poll timeout. */
#define UQ_OK 0
#define UQ_ERR_SHAPE (-1)
#define UQ_ERR_QUANT_TYPE (-2)
#define UQ_ERR_NONFINITE (-3)
#define UQ_ERR_DEVICE (-4)
#define UQ_ERR_TIMEOUT (-5)
#define UQ_ERR_CONTEXT (-6)
#define UQ_ERR_ARG (-7)
#define UQ_ERR_FORMAT (-8) /* malformed GGUF file; detail in the gguf_error out-parameter */

/* GGUF tensor kinds (ggml type ids, frontier_core.rs:53-58 plus Q3_K/Q4_K). */
#define UQ_KIND_F32 0u
#define UQ_KIND_Q8_0 8u
#define UQ_KIND_Q3_K 11u
#define UQ_KIND_Q4_K 12u
#define UQ_KIND_Q6_K 14u
#define UQ_KIND_IQ3_XXS 18u
#define UQ_KIND_IQ4_NL 20u
#define UQ_KIND_IQ4_XS 23u
#define UQ_KIND_BF16 30u

/* ---------------------------------------------------------------- context */
/* Replaces the GSP/RM channel bring-up that ends in llm::run's Gpu value
 * (driver/src/llm.rs:287-300): selects the HIP device and creates the stream. */
int uq_init(int device);
int uq_shutdown(void);
const char* uq_last_error(void);
/* Library stream as a hipStream_t (void* so the header needs no HIP includes). */
void* uq_stream(void);
int uq_sync(void);

/* GGUF row size of `n` values (frontier_core.rs:53-58 row_bytes); <0 on error. */
int64_t uq_row_bytes(uint32_t kind, int64_t n);
/* Free and total device memory of the context's GPU (hipMemGetInfo); the
 * capacity the reference's residency planning budgets against
 * (frontier_backend.rs:293-348, frontier_cache.rs:9-106). */
int uq_device_memory(size_t* free_bytes, size_t* total_bytes);

/* ---------------------------------------------------------------- weights */
typedef struct uq_weight* uq_weight_t;
/* Upload one GGUF tensor of m rows x n values (Tensor{n, m, typ}, llm.rs:63),
 * repack it on the device into the kernel layout, rebuild the GGUF bytes from
 * that layout and require a byte-for-byte match (llm.rs:187-200 upload
 * readback, gpu_prefill.rs:74-93 swizzle verify). kind: Q8_0, Q4_K, Q3_K for
 * the int8-activation linears below; F32, BF16, Q8_0, Q6_K, IQ3_XXS, IQ4_NL,
 * IQ4_XS for the fp32-activation reader (F32/BF16: n % 8 == 0). */
int uq_weight_upload(uint32_t kind, int64_t n, int64_t m, const void* gguf, size_t bytes, uq_weight_t* out);
int uq_weight_free(uq_weight_t w);
/* Device bytes held by the weight (repacked planes). */
int64_t uq_weight_bytes(uq_weight_t w);

/* ---------------------------------------------------------------- linears */
/* graph_quant + graph_linear (gpu_graph.rs:70-80) as one host call: y = W x,
 * x of n floats, y of m floats, host memory, synchronous. x is quantized per
 * 32 to int8 (quant_act, gpu_dp4a.cu:23-31) and the dot runs on int8
 * (linear_dp4a, gpu_dp4a.cu:40-52), the decode graph's arithmetic. Q8_0, Q4_K,
 * Q3_K weights; n % 32 == 0 (K-quants: % 256), n <= 16384, m <= 160000.
 * Non-finite x -> UQ_ERR_NONFINITE. The reference's Gpu::matvec computes on
 * fp32 x instead: its drop-in is uq_linear with a Q8_0 weight. */
int uq_matvec(uq_weight_t w, const float* x, int64_t n, float* y, int64_t m);
/* graph_linear over 1..3 weights sharing one quantized x (the decode graph's
 * q/k/v and gate/up groups, gpu_graph.rs:137-162), host memory. All-Q8_0
 * groups run as one job-table launch. */
int uq_batch(const uq_weight_t* ws, int count, const float* x, int64_t n, float* const* ys, const int64_t* ms);

/* Device forms (graph_quant / graph_linear, gpu_graph.rs:70-80). stream may be
 * NULL for the library stream. xq: n int8, xs: n/32 floats. */
int uq_quant_act_dev(const float* x, int64_t n, int8_t* xq, float* xs, void* stream);
int uq_matvec_q_dev(uq_weight_t w, const int8_t* xq, const float* xs, float* y, void* stream);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): uq_matvec on device pointers, x (n floats) -> y (m
 * floats) on `stream` (NULL: library stream), without synchronizing. The
 * quantized activation goes to a static device scratch of the library
 * (n <= 16384, else UQ_ERR_SHAPE); the call allocates and frees nothing. Every
 * call on one GPU shares that scratch: calls that overlap on one GPU (other
 * streams, other threads) race. Output equals uq_matvec's bit for bit; x is
 * not checked for non-finite values. */
int uq_matvec_static(uq_weight_t w, const float* x, float* y, void* stream);
/* gateup_dp4a (gpu_dp4a.cu:60-64): out[r] = silu(gate_r . x) * (up_r . x). */
int uq_gateup_q_dev(uq_weight_t gate, uq_weight_t up, const int8_t* xq, const float* xs, float* out, void* stream);

/* graph_linear over several weights as one launch (gpu_graph.rs:74-80, in the
 * job-table form of frontier_multi_matvec, kernels/frontier_quant.cu:79-93):
 * up to 8 Q8_0 weights of one input length
 * over one quantized x; w2s (may be NULL, entries may be NULL) pairs weight i
 * with an up matrix, ys[i] = silu(gate x) * (up x). Each output equals the
 * single-weight launch's bit for bit. */
int uq_matvec_table_dev(const uq_weight_t* ws, const uq_weight_t* w2s, int count, const int8_t* xq, const float* xs,
                        float* const* ys, void* stream);

/* Integer surfaces, host memory, synchronous. uq_quant_act: x (n floats) ->
 * q (n int8) + scale (n/32 floats) on the GPU (quant_act). uq_block_dots:
 * int32 per-block dots of W with the quantized x (Q8_0: m*(n/32) per 32-block,
 * Q4_K: m*(n/32) per 32 sub-block with q in 0..15, Q3_K: m*(n/16) per 16
 * sub-block with q3 in -4..3), the int32 sums of gpu_dp4a.cu:43-46 and
 * gpu_prefill.rs:111-115. */
int uq_quant_act(const float* x, int64_t n, int8_t* q, float* scale);
int uq_block_dots(uq_weight_t w, const float* x, int64_t n, int32_t* dots, int64_t count);

/* The prefill GEMM alone (prefill_gemm, gpu_prefill.cu:10-36; CPU check
 * gpu_prefill.rs:95-121): y[t][r] for `tokens` rows of pre-quantized
 * activations xq[t][n] with scales xs[t][n/32], host memory. Q8_0, m % 64. */
int uq_prefill_gemm(uq_weight_t w, const int8_t* xq, const float* xs, int64_t tokens, float* y);

/* Mean HIP-event time of the prefill GEMM on `tokens` synthetic activations
 * (w2 non-null: the fused gate/up pair), `reps` launches. Measurement aid. */
int uq_time_prefill_gemm(uq_weight_t w, uq_weight_t w2, int64_t tokens, int reps, double* ms);

/* Mean HIP-event time of the prefill's causal attention (the batched form of
 * fused_attention, gpu_attention.cu:2-26) over `tokens` synthetic queries at
 * positions 0.. against an fp16 KV cache of the same length, `reps` launches;
 * quant_out (head_dim 128): the epilogue writes the o GEMM's int8 planes, as
 * the model's prefill does. Measurement aid. */
int uq_time_prefill_attention(int32_t tokens, int32_t heads, int32_t kv_heads, int32_t head_dim, int quant_out,
                              int reps, double* ms);

/* ---------------------------------------------------------------- fp32-activation reader
 * The frontier backend's kernels (driver/kernels/frontier_quant.cu:12-93) for
 * its seven kinds, with fp32 activations. Each output is the exact sum of the
 * dequantized weights times x, rounded to f32 once; the reference's own check
 * allows 2e-4 + 2e-5 |ref| against an f32 sequential sum (frontier_gpu.rs:111). */

/* frontier_dequant (frontier_quant.cu:34-37) = dequantize (frontier_core.rs:73-106):
 * the n values of one GGUF byte run (nbytes == row_bytes(kind, n)) as f32, bit
 * for bit; host memory, synchronous. Q3_K/Q4_K -> UQ_ERR_QUANT_TYPE as there. */
int uq_dequantize(uint32_t kind, const void* bytes, size_t nbytes, int64_t n, float* out);

/* One entry of the FrontierJob table (frontier_quant.cu:71-78): weight, its
 * input (n floats) and output (m floats). */
typedef struct {
    uq_weight_t weight;
    const float* x;
    float* y;
} uq_linear_job;

/* Weights::linear (frontier_forward.rs:17; frontier_backend.rs:243) over
 * frontier_matvec (frontier_quant.cu:58-66): y = W x, host memory, synchronous.
 * Non-finite input or output -> UQ_ERR_NONFINITE (frontier_backend.rs:222,272);
 * Q3_K/Q4_K weights -> UQ_ERR_QUANT_TYPE.
 * With a Q8_0 weight this is also Gpu::matvec (llm.rs:246-273): matvec_q8 on
 * fp32 x (llm.rs:294-297), gated against the fp32 dequant dot at abs 0.002
 * (llm.rs:302-309). Its shape rule (llm.rs:248: typ 8, n % 32 == 0,
 * n <= 16384, m <= 160000) is the caller's check there and here.
 * Device staging is one library buffer grown to the largest call so far. */
int uq_linear(uq_weight_t w, const float* x, int64_t n, float* y, int64_t m);
/* Weights::batch (frontier_forward.rs:18; frontier_backend.rs:178-224): the jobs
 * (host x and y) in ONE launch, the frontier_multi_matvec of
 * frontier_quant.cu:79-93; bit-identical to uq_linear of each job.
 * With 1..3 Q8_0 jobs sharing one x this is Gpu::batch (llm.rs:226-245), whose
 * prebuilt jobs copy the fp32 matvec_q8 launch (llm.rs:202-214). */
int uq_linear_batch(const uq_linear_job* jobs, int count);
/* Device forms on `stream` (NULL: library stream), no synchronization; x must
 * be 16-byte aligned. */
int uq_linear_dev(uq_weight_t w, const float* x, float* y, void* stream);
int uq_linear_multi_dev(const uq_linear_job* jobs, int count, void* stream);
/* Measurement aid (no reference counterpart): `reps` rounds, after `warmup`
 * untimed ones, of one uq_linear_dev launch per weight in turn (zero x, each
 * weight its own output); total_ms = HIP-event time of the timed rounds. */
int uq_time_linear(const uq_weight_t* ws, int count, int reps, int warmup, double* total_ms);
/* Measurement aid (no reference counterpart): the job tables jobs[0..sizes[0]),
 * then the next sizes[1] jobs, ..., each one uq_linear_multi_dev launch
 * (device x/y), repeated reps times after one untimed round; total_ms =
 * HIP-event time of the timed rounds. */
int uq_time_linear_tables(const uq_linear_job* jobs, const int* sizes, int ntables, int reps, double* total_ms);

/* ---------------------------------------------------------------- memory + timing
 * Small helpers so harnesses need no other GPU runtime binding. */
int uq_dev_alloc(size_t bytes, void** ptr);
int uq_dev_free(void* ptr);
int uq_memcpy_h2d(void* dst, const void* src, size_t bytes);
int uq_memcpy_d2h(void* dst, const void* src, size_t bytes);
/* Times `reps` rounds of matvecs over `count` weights (each weight its own
 * input/output), all on the library stream, after `warmup` untimed rounds.
 * Per-launch HIP event pairs are recorded around launches of weight index
 * `probe` (or none if probe < 0). total_ms: whole timed region; probe_ms: mean
 * duration of the probed launch. pairs[i] != 0 marks weight i as the gate of a
 * gate/up pair with weight i+1 (one fused launch). */
int uq_time_matvecs(const uq_weight_t* ws, const int* pairs, int count, int64_t max_n, int reps, int warmup,
                    int probe, double* total_ms, double* probe_ms);

/* The same measurement with consecutive Q8_0 weights of one input length (up
 * to 8) launched as one job table (the batch of llm.rs:226-245); each output as
 * uq_matvec_q_dev gives it. */
int uq_time_matvec_tables(const uq_weight_t* ws, const int* pairs, int count, int64_t max_n, int reps, int warmup,
                          double* total_ms);

/* Achievable-bandwidth probe (no reference counterpart; measurement aid): a
 * streaming read of `bytes` and a copy of `bytes` (read + write counted),
 * `reps` launches each, GB/s from HIP events. */
int uq_probe_bandwidth(int64_t bytes, int reps, double* read_gbs, double* copy_gbs);

/* Matrix-core throughput probe (no reference counterpart; measurement aid):
 * independent chains of one MFMA on register operands, 16 waves per CU, rate
 * from HIP events. kind 0: v_mfma_i32_16x16x32_i8 (tera int8 ops/s), 1:
 * v_mfma_f32_16x16x32_f16 (TFLOP/s), 2: v_mfma_f64_16x16x4_f64 (TFLOP/s).
 * One wave per SIMD, rate counted as the MFMA work of the iterations (also
 * where only the VALU part runs): 3: fp64 MFMAs alone, 4: with an fp16 ->
 * double B-operand conversion per MFMA, 5: those conversions alone; 6: int8
 * MFMAs alone, 7: beside a convert / scale product / fma per f32 accumulator
 * (the prefill GEMM's rescale), 8: that rescale alone. Whether a kind's VALU
 * work overlaps the matrix core: 1/rate(4) vs 1/rate(3) + 1/rate(5).
 * 16 waves per CU again: 9: v_mfma_i32_32x32x32_i8, 10: v_mfma_i32_16x16x64_i8
 * (tera int8 ops/s). */
int uq_probe_mfma(int kind, double* tera_ops);

/* ---------------------------------------------------------------- Qwen2 dense decoder */
/* Model shape constants of driver/src/llm.rs:314-321 (DIM, HIDDEN, KV, HEAD,
 * SEQ, LAYERS) as a runtime description. */
typedef struct {
    int32_t layers, dim, hidden, heads, kv_heads, head_dim, vocab, max_seq;
    float eps, theta;
} uq_qwen2_config;
typedef struct uq_model* uq_model_t;

/* Arena allocation of init_graph (gpu_graph.rs:81-87). Requires uq_init. */
int uq_model_create(const uq_qwen2_config* cfg, uq_model_t* out);
int uq_model_free(uq_model_t m);
/* upload_weights (llm.rs:157-201) for one GGUF tensor by name
 * ("token_embd.weight", "output.weight", "output_norm.weight",
 * "blk.N.attn_{q,k,v,output}.weight", "blk.N.ffn_{gate,up,down}.weight",
 * "blk.N.{attn,ffn}_norm.weight", "blk.N.attn_{q,k,v}.bias"): Q8_0 matrices
 * (n columns, rows) or F32 vectors (rows == 1). Biases are optional. */
int uq_model_set_tensor(uq_model_t m, const char* name, uint32_t kind, int64_t n, int64_t rows, const void* data,
                        size_t bytes);
/* init_graph (gpu_graph.rs:81-169): checks every tensor, builds the RoPE table
 * (gpu_graph.rs:131-133) and captures one decode step into a hipGraph. */
int uq_model_prepare(uq_model_t m);
/* forward_gpu (gpu_graph.rs:170-197): one decode step of `token` at `pos`,
 * writes the greedy next id; non-finite logits -> UQ_ERR_NONFINITE. */
int uq_decode_step(uq_model_t m, uint32_t token, int pos, uint32_t* next);
/* The decode loop of generate_one (llm.rs:422-428) with the greedy id fed back
 * on the device: `steps` graph launches from (token, pos), tokens[i] = id
 * produced at position pos+i; ms (optional) = hipEvent time of the launches. */
int uq_decode_run(uq_model_t m, uint32_t token, int pos, int steps, uint32_t* tokens, double* ms);
/* Prompt ingestion through the decode graph, one launch per prompt token at
 * positions pos..pos+count-1 (the per-token forward of llm.rs:339-388); next =
 * greedy id after the last prompt token. */
int uq_prompt_tokens(uq_model_t m, const uint32_t* tokens, int count, int pos, uint32_t* next);
/* prepare_prefill + run_prefill (gpu_prefill.rs:122-157): the prompt at
 * positions 0..count-1 through int8-MFMA GEMMs and causal attention, filling
 * the fp16 KV cache; next = greedy id after the last prompt token. The decode
 * step continues at pos = count. count <= min(max_seq, 1024). */
int uq_prefill(uq_model_t m, const uint32_t* tokens, int count, uint32_t* next);
/* generate_one (llm.rs:402-428): prefill of the prompt (count tokens), then
 * up to max_new greedy steps. Before each step the current id is compared
 * with the stop ids (the reference's 151645 / 151643); a stop id ends the
 * run (*ended = 1) and is not emitted. out[0..*generated) are the emitted ids;
 * count + max_new < max_seq. prefill_ms / decode_ms (optional): host-clock
 * time of each phase, each ending with its ids on the host. */
int uq_generate(uq_model_t m, const uint32_t* prompt, int count, int max_new, const uint32_t* stop, int nstop,
                uint32_t* out, int* generated, int* ended, double* prefill_ms, double* decode_ms);
/* LOGITS readback of verify_gpu_greedy (gpu_graph.rs:14-23). */
int uq_model_logits(uq_model_t m, float* out, int64_t n);
/* fp16 KV cache readback of positions [0, count) of one layer ([count][kv*hd]). */
int uq_model_kv(uq_model_t m, int layer, int count, uint16_t* keys, uint16_t* values);

/* ---------------------------------------------------------------- MoE expert FFN */
/* Forward::ffn (driver/src/frontier_forward.rs:164-199) for one token: softmax
 * routing over `experts` router logits, stable top-k (score descending, id
 * ascending), weights score/sum(top-k); per selected expert and for the shared
 * expert down(silu(gate x) * (up x)) with int8 activations per 32; combine in
 * rank order, shared expert weighted by sigmoid(gate_inp . x). The expert
 * matrices live in one HBM-resident bank per projection; the routing result
 * stays on the device (the FrontierJob table of frontier_quant.cu:71-93). */
typedef struct uq_moe* uq_moe_t;
int uq_moe_create(int32_t dim, int32_t ff, int32_t experts, int32_t top_k, uint32_t expert_kind, uq_moe_t* out);
int uq_moe_free(uq_moe_t m);
/* GGUF bytes of expert e: gate and up (ff rows x dim), down (dim rows x ff). */
int uq_moe_set_expert(uq_moe_t m, int32_t e, const void* gate, const void* up, const void* down);
/* Shared expert (ffn_{gate,up,down}_shexp) and its f32 gate vector
 * ffn_gate_inp_shexp of dim values (NULL: weight 1). */
int uq_moe_set_shared(uq_moe_t m, uint32_t kind, const void* gate, const void* up, const void* down,
                      const float* gate_inp);
/* The layer's shape as created. */
int uq_moe_info(uq_moe_t m, int32_t* dim, int32_t* ff, int32_t* experts, int32_t* top_k, uint32_t* expert_kind);
/* Host-memory call: x (dim), router logits (experts) -> out (dim); optional
 * ids/weights (top_k) of the routing. Non-finite input -> UQ_ERR_NONFINITE. */
int uq_moe_ffn(uq_moe_t m, const float* x, const float* router_logits, float* out, int32_t* ids, float* weights);
/* Device-pointer form on `stream` (NULL: library stream), no synchronization;
 * x must be 16-byte aligned (UQ_ERR_ARG otherwise). */
int uq_moe_ffn_dev(uq_moe_t m, const float* x, const float* router_logits, float* out, void* stream);
/* `steps` tokens back to back on the library stream, device arrays x[steps][dim],
 * logits[steps][experts], out[steps][dim]; ms = HIP-event time of the launches. */
int uq_moe_run(uq_moe_t m, const float* xs, const float* logits, float* outs, int steps, double* ms);

/* ---------------------------------------------------------------- GGUF files */
/* Bounded GGUF v3 directory parser, Shard::parse (driver/src/frontier_gguf.rs:
 * 145-200): the directory must fit a 16 MiB prefix; tensor bodies stay on
 * storage. Failures return UQ_ERR_FORMAT and one of the reference's error
 * categories (frontier_gguf.rs:7-8) in *gguf_error. */
#define UQ_GGUF_TRUNCATED 1
#define UQ_GGUF_MAGIC 2
#define UQ_GGUF_VERSION 3
#define UQ_GGUF_LIMIT 4
#define UQ_GGUF_TYPE 5
#define UQ_GGUF_UTF8 6
#define UQ_GGUF_ALIGNMENT 7
#define UQ_GGUF_SHAPE 8
#define UQ_GGUF_OVERFLOW 9
#define UQ_GGUF_TENSOR_BOUNDS 10
#define UQ_GGUF_OVERLAP 11
#define UQ_GGUF_DUPLICATE 12
#define UQ_GGUF_MISSING 13
#define UQ_GGUF_SPLIT 14
typedef struct uq_gguf* uq_gguf_t;
/* Shard::parse(prefix, logical_bytes): directory from `len` bytes of a file of
 * `logical_bytes` bytes (no file access; tensor offsets are absolute). */
int uq_gguf_parse(const void* prefix, size_t len, uint64_t logical_bytes, uq_gguf_t* out, int* gguf_error);
/* Opens a file: parses its first min(size, 16 MiB) bytes with logical_bytes =
 * the file size, and keeps the path for uq_model_load_gguf. */
int uq_gguf_open(const char* path, uq_gguf_t* out, int* gguf_error);
int uq_gguf_free(uq_gguf_t g);
int64_t uq_gguf_tensor_count(uq_gguf_t g);
uint64_t uq_gguf_data_offset(uq_gguf_t g);
/* split.no, split.count, split.tensors.count (defaults 0, 1, tensor count). */
int uq_gguf_split_info(uq_gguf_t g, uint64_t* split_no, uint64_t* split_count, uint64_t* total_tensors);
/* Tensor `index`: name (valid while g lives), ggml kind, rank, dims[4] (unused
 * dims 1), absolute file offset and byte size (Tensor, frontier_gguf.rs:95-99). */
int uq_gguf_tensor_info(uq_gguf_t g, int64_t index, const char** name, uint32_t* kind, int32_t* rank, uint64_t* dims,
                        uint64_t* offset, uint64_t* bytes);
/* Index of the tensor called `name`, or -1 (Shard::tensor). */
int64_t uq_gguf_find_tensor(uq_gguf_t g, const char* name);
/* Metadata values (Value::unsigned for u8/u16/u32/u64, Value::float, Value::string,
 * frontier_gguf.rs:44-66); the string is not NUL-terminated. */
int uq_gguf_meta_u64(uq_gguf_t g, const char* key, uint64_t* out);
int uq_gguf_meta_f32(uq_gguf_t g, const char* key, float* out);
int uq_gguf_meta_str(uq_gguf_t g, const char* key, const char** out, uint64_t* len);
int uq_gguf_meta_array(uq_gguf_t g, const char* key, uint32_t* elem_kind, uint64_t* count);
/* Element `index` of a string-array value (e.g. tokenizer.ggml.tokens):
 * pointer into the parsed directory and its byte length. */
int uq_gguf_meta_array_str(uq_gguf_t g, const char* key, uint64_t index, const char** out, uint64_t* len);
/* Tensor::rows (frontier_gguf.rs:86-94): absolute file range of `count`
 * contiguous rows of tensor `index` from row `start`; count 0 or rows past the
 * end -> UQ_ERR_FORMAT with UQ_GGUF_TENSOR_BOUNDS (UQ_GGUF_OVERFLOW on
 * overflow). */
int uq_gguf_tensor_rows(uq_gguf_t g, int64_t index, uint64_t start, uint64_t count, uint64_t* offset, uint64_t* bytes,
                        int* gguf_error);
/* Tensor::expert (frontier_gguf.rs:95-98): the rows of expert `expert` of a
 * rank-3 [n, rows, experts] tensor; another rank or expert >= dims[2] ->
 * UQ_GGUF_SHAPE. */
int uq_gguf_tensor_expert(uq_gguf_t g, int64_t index, uint32_t expert, uint64_t* offset, uint64_t* bytes,
                          int* gguf_error);

/* ModelIndex (frontier_gguf.rs:101-137) over the directories of a split
 * model: ModelIndex::new orders the shards by split.no and requires split.no
 * 0..count-1, split.count == count and one split.tensors.count on every shard
 * (else UQ_GGUF_SPLIT), no tensor name twice (UQ_GGUF_DUPLICATE), and as many
 * tensors as split.tensors.count (UQ_GGUF_SPLIT). The index keeps the shard
 * handles, which must outlive it. */
typedef struct uq_gguf_index* uq_gguf_index_t;
int uq_gguf_index_create(const uq_gguf_t* shards, int count, uq_gguf_index_t* out, int* gguf_error);
int uq_gguf_index_free(uq_gguf_index_t ix);
int uq_gguf_index_shard_count(uq_gguf_index_t ix);
/* Shard i in split.no order (NULL when out of range). */
uq_gguf_t uq_gguf_index_shard(uq_gguf_index_t ix, int i);
/* ModelIndex::tensor: the shard (split.no order) and index of tensor `name`;
 * UQ_GGUF_MISSING when no shard holds it. */
int uq_gguf_index_find(uq_gguf_index_t ix, const char* name, int* shard, int64_t* index, int* gguf_error);
/* ModelIndex::inventory: on-disk bytes of [other tensors,
 * per_layer_token_embd.weight, *_exps.weight]. */
int uq_gguf_index_inventory(uq_gguf_index_t ix, uint64_t* bytes3, int* gguf_error);
/* A tensor of a file-backed shard as a device weight (uq_weight_upload of its
 * bytes: n = dims[0], one row per remaining dim), or with expert >= 0 the
 * rows of that expert of a rank-3 tensor (Backend::expert's byte range,
 * frontier_backend.rs:98-128). Any kind uq_weight_upload takes. */
int uq_gguf_load_weight(uq_gguf_t g, int64_t index, int32_t expert, uq_weight_t* out);
/* The expert bank of MoE layer `layer` from a split model: every expert of
 * blk.L.ffn_{gate,up,down}_exps.weight (rank 3, the bank's kind and shape)
 * and the shared expert blk.L.ffn_{gate,up,down}_shexp.weight with the
 * optional f32 blk.L.ffn_gate_inp_shexp.weight, loaded into `m` as
 * uq_moe_set_expert / uq_moe_set_shared would. Fails with UQ_ERR_DEVICE before
 * reading when twice the layer's bytes exceed the free HBM. */
int uq_moe_load_gguf(uq_moe_t m, uq_gguf_index_t ix, int32_t layer);
/* Model::text (driver/src/llm.rs:87-99): the bytes of token `id` from the
 * GPT-2 byte-level string in tokenizer.ggml.tokens. len = bytes needed; the
 * call fails with UQ_ERR_ARG (len still set) when cap is smaller. */
int uq_gguf_token_text(uq_gguf_t g, uint32_t id, uint8_t* out, uint64_t cap, uint64_t* len);
/* Qwen2 shape constants from qwen2.* metadata and token_embd.weight (the
 * constants llm.rs:314-321 hard-codes); max_seq <= 0 takes context_length. */
int uq_gguf_qwen2_config(uq_gguf_t g, int32_t max_seq, uq_qwen2_config* cfg);
/* upload_weights (llm.rs:157-201) from a GGUF file: every blk.* tensor plus
 * token_embd, output_norm and output (token_embd when the file ties them) into
 * the model, read from the file the handle was opened from. */
int uq_model_load_gguf(uq_model_t m, uq_gguf_t g);

#ifdef __cplusplus
}
#endif
#endif
