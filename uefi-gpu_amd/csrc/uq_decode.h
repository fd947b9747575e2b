// Argument block of the residual + RMSNorm + quant prologues (and the layer-0
// embedding row) that the decode-step and prefill kernels run inline.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace uq {

// Residual + RMSNorm + block-32 quant of one activation vector:
// x = embed ? dequant(token row) : x_in (+ residual); x_out = x (optional);
// y = (x * (1/sqrt(mean(x^2) + eps))) * gamma; y quantized per 32.
struct NormQuantArgs {
    const float* x;          // residual stream in [dim]
    const float* residual;   // added when non-null
    const float* gamma;      // RMSNorm weight [dim]
    float* x_out;            // summed residual out (written by one workgroup)
    int8_t* xq;              // quantized output (global), when the kernel writes it out
    float* xs;
    const int8_t* embed_qs;  // when set: x = dequant(token row) (Q8_0 planes)
    const uint16_t* embed_d;
    const uint32_t* token;
    int dim;
    float eps;
};

}  // namespace uq
