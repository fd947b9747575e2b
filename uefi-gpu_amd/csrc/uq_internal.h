// Internal host-side declarations shared by the library's translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>

namespace uq {

enum Status : int {
    OK = 0,
    ERR_SHAPE = -1,       // frontier_forward.rs:10 Error::Shape
    ERR_QUANT_TYPE = -2,  // frontier_core.rs:37 Error::QuantType
    ERR_NONFINITE = -3,   // Error::NonFinite
    ERR_DEVICE = -4,      // Error::Backend (device call failed)
    ERR_TIMEOUT = -5,     // llm.rs:267-269 bounded poll expired
    ERR_CONTEXT = -6,     // Error::Context (position beyond the cache)
    ERR_ARG = -7,         // null pointer / bad handle / wrong state
    ERR_FORMAT = -8,      // malformed GGUF file (frontier_gguf.rs:7-8 Error)
};

enum Kind : uint32_t {
    KIND_F32 = 0,
    KIND_Q8_0 = 8,
    KIND_Q3_K = 11,
    KIND_Q4_K = 12,
    KIND_Q6_K = 14,
    KIND_IQ3_XXS = 18,
    KIND_IQ4_NL = 20,
    KIND_IQ4_XS = 23,
    KIND_BF16 = 30,
};

int set_error(int status, const std::string& msg);
#define UQ_CHECK_HIP(call)                                                        \
    do {                                                                          \
        hipError_t e_ = (call);                                                   \
        if (e_ != hipSuccess)                                                     \
            return ::uq::set_error(::uq::ERR_DEVICE, std::string(#call) + ": " +  \
                                                     hipGetErrorString(e_));      \
    } while (0)

int64_t row_bytes(uint32_t kind, int64_t n);  // GGUF bytes of one row, <0 if invalid

// Device-resident weight. The frontier kinds (F32, BF16, Q6_K, IQ3_XXS,
// IQ4_NL, IQ4_XS) use the planes of their FrontierLayout: qs = body units,
// sc = aux bytes, d = fp16 block scales. Q8_0 is split into an int8 plane qs[m][n] and an
// fp16 scale plane d[m][n/32]; Q4_K and Q3_K use the unit planes of Q4K /
// Q3K (qs, sc, d); lm_head-sized Q3_K weights use the row-block layout of
// Q3KSB in qs alone.
struct Weight {
    uint32_t kind = 0;
    int64_t n = 0, m = 0;   // n = K (input length), m = N (output rows)
    void* alloc = nullptr;  // single device allocation owning the planes
    size_t alloc_bytes = 0;
    const int8_t* qs = nullptr;    // Q8_0 quants / Q3_K quants / Q4_K superblocks
    const uint16_t* d = nullptr;   // Q8_0 / Q3_K fp16 scales
    const uint8_t* sc = nullptr;   // Q3_K packed scales
    int64_t gguf_bytes = 0;        // bytes of the original GGUF tensor
    // Q3_K in the row-block layout (uq_units.h, SbGeom): lane slots and rows
    // per block, 0 for the unit planes
    int sb_lb = 0, sb_rb = 0;
};

// Compute units of the current device (queried once).
int cu_count();

// Device staging of the host-pointer fp32 calls: one buffer per context,
// grown on demand and never shrunk, so repeated calls of the same sizes
// allocate nothing. Valid until the next call that asks for more bytes.
int staging_buffer(size_t bytes, void** out);

int upload_weight(uint32_t kind, int64_t n, int64_t m, const void* gguf, size_t bytes, Weight& out, bool bank);

// Split of one GGUF block of a frontier kind into three planes (body, aux,
// fp16 scale): map[o] = plane << 12 | offset of source byte o within that
// plane's per-block slice of plane_bytes[plane] bytes (uq_frontier.hip).
struct FrontierLayout {
    int block_vals, block_bytes;
    int plane_bytes[3];
    uint16_t map[256];
};
bool frontier_layout(uint32_t kind, FrontierLayout& L);
void launch_layout_repack(const uint8_t* src, int64_t blocks, const FrontierLayout& L, uint8_t* const planes[3],
                          hipStream_t s);
void launch_layout_verify(const uint8_t* src, int64_t blocks, const FrontierLayout& L, uint8_t* const planes[3],
                          unsigned* bad, hipStream_t s);

// ---- kernel launchers (uq_matvec.hip) ----
void launch_quant_act(const float* x, int64_t n, int8_t* xq, float* xs, hipStream_t s);
void launch_q8_repack(const uint8_t* gguf, int64_t rows, int64_t nb, int8_t* qs, uint16_t* d, hipStream_t s);
void launch_q8_verify(const int8_t* qs, const uint16_t* d, const uint8_t* gguf, int64_t rows, int64_t nb,
                      unsigned* mismatches, hipStream_t s);
void launch_q4k_repack(const uint8_t* gguf, int64_t blocks, int64_t spr, int8_t* q, uint8_t* scm, uint32_t* dm,
                       hipStream_t s);
void launch_q4k_verify(const int8_t* q, const uint8_t* scm, const uint32_t* dm, const uint8_t* gguf, int64_t blocks,
                       int64_t spr, unsigned* bad, hipStream_t s);
void launch_q3k_repack(const uint8_t* gguf, int64_t blocks, int8_t* q, int8_t* sc, uint16_t* d, hipStream_t s);
void launch_q3k_verify(const int8_t* q, const int8_t* sc, const uint16_t* d, const uint8_t* gguf, int64_t blocks,
                       unsigned* mismatches, hipStream_t s);
// Q3_K into the row-block layout (lb slots, rb rows per block) at dst
// (zeroed beforehand), then the byte-for-byte rebuild check into *bad.
void launch_sb_repack(uint32_t kind, const uint8_t* gguf, int64_t n, int64_t m, int lb, int rb, uint8_t* dst,
                      unsigned* bad, hipStream_t s);
// y[m] = W x for any kind; gate/up fusion writes silu(gate)*up when w2 != null.
int launch_matvec(const Weight& w, const Weight* w2, const int8_t* xq, const float* xs, float* y, hipStream_t s);
int launch_block_dots(const Weight& w, const int8_t* xq, int32_t* dots, hipStream_t s);
// Up to 8 Q8_0 weights of one input length (w2s[i] non-null: gate/up pair) in
// one launch over a shared quantized x; each output as launch_matvec gives it.
int launch_matvec_multi(const Weight* const* ws, const Weight* const* w2s, float* const* ys, int count,
                        const int8_t* xq, const float* xs, hipStream_t s);

}  // namespace uq

// The opaque handle of include/uq.h.
struct uq_weight {
    uq::Weight w;
};
