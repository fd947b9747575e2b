// Host-side state of the Qwen2 dense decoder (uq_model.hip).
#pragma once
#include "uq_internal.h"
#include "../../include/uq.h"

#include <map>
#include <string>
#include <vector>

namespace uq {

struct LayerDev {
    Weight qkv;  // q|k|v rows of one layer in one Q8_0 weight
    // fp16 weight scales transposed to [k/32][rows] for the prefill GEMM
    float *qkv_dt = nullptr, *o_dt = nullptr, *g_dt = nullptr, *u_dt = nullptr, *d_dt = nullptr;
    // the prefill's q|k|v copy with the RoPE partners adjacent (PfRopeEpi):
    // int8 rows, and the permuted q|k|v bias; qkv_dt is in the same row order
    int8_t* qkv_pq = nullptr;
    float* qkv_pb = nullptr;
};

struct Model {
    uq_qwen2_config cfg{};
    hipStream_t stream = nullptr;
    bool prepared = false;
    bool eager = false;
    std::map<std::string, uq_weight_t> q8;
    std::map<std::string, float*> f32;
    std::map<std::string, int64_t> f32_len;
    std::vector<LayerDev> layers;
    std::vector<void*> owned;

    float *R0 = nullptr, *R1 = nullptr, *TMP = nullptr, *XN = nullptr, *QKV = nullptr, *ATT = nullptr, *GATE = nullptr,
          *LOGITS = nullptr, *XS = nullptr, *trig = nullptr;
    int8_t* XQ = nullptr;  // quantized dim-sized activation (lm_head input)
    uint16_t *kcache = nullptr, *vcache = nullptr;
    uint32_t *token = nullptr, *history = nullptr, *result = nullptr;
    int* pos = nullptr;
    uint32_t* partial = nullptr;
    float *SC = nullptr, *CM = nullptr;  // attention scores [heads][max_seq], chunk maxima [heads][ATT_SPLIT]
    double* ACC = nullptr;               // attention output accumulator [heads*hd]
    uint32_t host_io[4] = {0, 0, 0, 0};

    // prefill arenas, sized for pcap tokens (padded to the GEMM tile)
    int pcap = 0;
    float *PX = nullptr, *PTMP = nullptr, *PY = nullptr, *PATT = nullptr, *PG = nullptr, *PXST = nullptr;
    int8_t* PXQ = nullptr;
    uint32_t* PTOK = nullptr;

    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;

    ~Model();
    int fail(int st, const std::string& msg);
    const Weight* weight(const std::string& name) const;
    const float* vec(const std::string& name) const;
    int check_shapes();
    int build_qkv(int l);
    template <class T>
    int alloc(T** p, size_t count);
    int build_buffers();
    int enqueue_step(hipStream_t s);
    int prepare();
    int set_position(uint32_t tok, int p);
    int launch_step();
    int build_prefill();
    int prefill(const uint32_t* tokens, int n, uint32_t* next);
};

}  // namespace uq
