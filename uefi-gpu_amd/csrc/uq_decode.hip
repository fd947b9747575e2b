// Token embedding + residual + RMSNorm + block-32 quant in one workgroup
// (embedding_q8, gpu_embedding.cu:3-9; fused_resnorm_quant,
// gpu_norm_quant.cu:3-19; quant_act, gpu_dp4a.cu:23-31). The token is read
// from device memory so that one captured graph serves every step (the
// reference patches it into its push buffer per token, gpu_graph.rs:170-178).
#include "uq_device.h"
#include "uq_decode.h"
#include "uq_blockops.h"

namespace uq {
namespace {

__global__ __launch_bounds__(NQ_WG) void k_resnorm_quant(NormQuantArgs a) {
    __shared__ double red_d[NQ_WG / 64];
    norm_quant<NQ_WG>(a, true, a.xq, a.xs, red_d);
}

}  // namespace

void launch_resnorm_quant(const NormQuantArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_resnorm_quant, dim3(1), dim3(NQ_WG), 0, s, a);
}

}  // namespace uq
