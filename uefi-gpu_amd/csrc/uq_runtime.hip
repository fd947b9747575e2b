// Host runtime of the library: process context, device-resident weights and
// the synchronous linear calls of the reference's `Gpu` (driver/src/llm.rs:110-273).
//
// The reference submits hand-packed QMDs through a GPFIFO and polls sysmem
// semaphores; here one HIP stream per process carries every launch and
// hipStreamSynchronize is the completion poll.
#include "uq_internal.h"
#include "uq_units.h"
#include "../../include/uq.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

// Scratch of uq_matvec_static: one call's quantized activation, the int8
// codes of up to STATIC_MAX_N values followed by their f32 block scales. A
// file-scope device array, so that call allocates nothing; every device the
// library runs on holds its own copy until the process ends. Host code never
// uses the array's name as an address: uq_init looks up the device address
// (hipGetSymbolAddress) and keeps it per device.
#define UQ_STATIC_MAX_N 16384
static __device__ __align__(256) int8_t scratch[UQ_STATIC_MAX_N + UQ_STATIC_MAX_N / 32 * 4];

namespace uq {

namespace {
thread_local std::string g_error;

constexpr int MAX_DEVICES = 64;
void* g_scratch[MAX_DEVICES];  // device address of `scratch` per device, set by uq_init

struct Context {
    bool ready = false;
    int device = -1;
    hipStream_t stream = nullptr;
    // staging for the host-pointer linears: x, quantized x, outputs
    float* dx = nullptr;
    int8_t* dxq = nullptr;
    float* dxs = nullptr;
    float* dy = nullptr;
    size_t y_cap = 0;
    unsigned* dcount = nullptr;
    // staging of the fp32-activation host calls (uq_linear*, uq_dequantize):
    // grown on demand, never shrunk
    void* stage = nullptr;
    size_t stage_cap = 0;
};
Context g_ctx;

constexpr int64_t MAX_N = 16384;    // llm.rs:248 n<=16384
constexpr int64_t MAX_M = 160000;   // llm.rs:248 m<=160000
}  // namespace

int set_error(int status, const std::string& msg) {
    g_error = msg;
    return status;
}

int64_t row_bytes(uint32_t kind, int64_t n) {
    int64_t block, bytes;
    switch (kind) {
    case KIND_F32: block = 1; bytes = 4; break;
    case KIND_Q8_0: block = 32; bytes = 34; break;
    case KIND_Q4_K: block = 256; bytes = 144; break;
    case KIND_Q3_K: block = 256; bytes = 110; break;
    case KIND_Q6_K: block = 256; bytes = 210; break;
    case KIND_IQ3_XXS: block = 256; bytes = 98; break;
    case KIND_IQ4_NL: block = 32; bytes = 18; break;
    case KIND_IQ4_XS: block = 256; bytes = 136; break;
    case KIND_BF16: block = 1; bytes = 2; break;
    default: return ERR_QUANT_TYPE;
    }
    if (n <= 0 || n % block) return ERR_SHAPE;
    return n / block * bytes;
}

static int require_ctx() {
    if (!g_ctx.ready) return set_error(ERR_ARG, "uq_init has not been called");
    return OK;
}

static int ensure_y(size_t m) {
    if (m <= g_ctx.y_cap) return OK;
    if (g_ctx.dy) UQ_CHECK_HIP(hipFree(g_ctx.dy));
    g_ctx.dy = nullptr;
    UQ_CHECK_HIP(hipMalloc(&g_ctx.dy, sizeof(float) * 3 * m));
    g_ctx.y_cap = m;
    return OK;
}

static hipStream_t pick(void* s) { return s ? (hipStream_t)s : g_ctx.stream; }

int staging_buffer(size_t bytes, void** out) {
    if (!g_ctx.ready) return set_error(ERR_ARG, "uq_init has not been called");
    if (bytes > g_ctx.stage_cap) {
        // the previous buffer may still be read by enqueued copies
        size_t cap = std::max(bytes, 2 * g_ctx.stage_cap);
        cap = (cap + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);
        UQ_CHECK_HIP(hipStreamSynchronize(g_ctx.stream));
        if (g_ctx.stage) UQ_CHECK_HIP(hipFree(g_ctx.stage));
        g_ctx.stage = nullptr;
        g_ctx.stage_cap = 0;
        UQ_CHECK_HIP(hipMalloc(&g_ctx.stage, cap));
        g_ctx.stage_cap = cap;
    }
    *out = g_ctx.stage;
    return OK;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace uq

using namespace uq;

extern "C" {

const char* uq_last_error(void) { return uq::g_error.c_str(); }

int uq_init(int device) {
    if (g_ctx.ready) {
        if (g_ctx.device == device) return OK;
        return set_error(ERR_ARG, "uq_init: already initialised on another device");
    }
    int count = 0;
    UQ_CHECK_HIP(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) return set_error(ERR_ARG, "uq_init: no such device");
    UQ_CHECK_HIP(hipSetDevice(device));
    if (device < MAX_DEVICES && !g_scratch[device]) {
        void* p = nullptr;
        UQ_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return set_error(ERR_DEVICE, "uq_init: no device address for the static scratch");
        g_scratch[device] = p;
    }
    UQ_CHECK_HIP(hipStreamCreateWithFlags(&g_ctx.stream, hipStreamNonBlocking));
    UQ_CHECK_HIP(hipMalloc(&g_ctx.dx, sizeof(float) * MAX_N));
    UQ_CHECK_HIP(hipMalloc(&g_ctx.dxq, MAX_N));
    UQ_CHECK_HIP(hipMalloc(&g_ctx.dxs, sizeof(float) * (MAX_N / 32)));
    UQ_CHECK_HIP(hipMalloc(&g_ctx.dcount, sizeof(unsigned) * 4));
    g_ctx.device = device;
    g_ctx.ready = true;
    return OK;
}

int uq_shutdown(void) {
    if (!g_ctx.ready) return OK;
    hipStreamSynchronize(g_ctx.stream);
    hipFree(g_ctx.dx);
    hipFree(g_ctx.dxq);
    hipFree(g_ctx.dxs);
    hipFree(g_ctx.dy);
    hipFree(g_ctx.dcount);
    if (g_ctx.stage) hipFree(g_ctx.stage);
    hipStreamDestroy(g_ctx.stream);
    g_ctx = Context{};
    return OK;
}

void* uq_stream(void) { return (void*)g_ctx.stream; }

int uq_sync(void) {
    if (int rc = require_ctx()) return rc;
    UQ_CHECK_HIP(hipStreamSynchronize(g_ctx.stream));
    return OK;
}

int64_t uq_row_bytes(uint32_t kind, int64_t n) { return uq::row_bytes(kind, n); }

int uq_device_memory(size_t* free_bytes, size_t* total_bytes) {
    if (int rc = require_ctx()) return rc;
    size_t f = 0, t = 0;
    UQ_CHECK_HIP(hipMemGetInfo(&f, &t));
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return OK;
}

}  // extern "C"

namespace uq {
// Frontier kinds: the GGUF blocks are split into their planes on the device
// and every source byte is compared with its place in the planes.
static int upload_split(uint32_t kind, int64_t n, int64_t m, const void* gguf, int64_t rb, const FrontierLayout& L,
                        Weight& out) {
    hipStream_t s = g_ctx.stream;
    const int64_t blocks = n / L.block_vals * m;
    size_t off[3], total = 0;
    for (int p = 0; p < 3; p++) {
        off[p] = total;
        total += align256((size_t)(blocks * L.plane_bytes[p]));
    }
    Weight w;
    w.kind = kind;
    w.n = n;
    w.m = m;
    w.gguf_bytes = rb * m;
    UQ_CHECK_HIP(hipMalloc(&w.alloc, std::max<size_t>(total, 256)));
    w.alloc_bytes = total;
    uint8_t* base = (uint8_t*)w.alloc;
    uint8_t* planes[3] = {base + off[0], base + off[1], base + off[2]};
    w.qs = (const int8_t*)planes[0];
    w.sc = L.plane_bytes[1] ? planes[1] : nullptr;
    w.d = L.plane_bytes[2] ? (const uint16_t*)planes[2] : nullptr;
    void* staging = nullptr;
    hipError_t e = hipMalloc(&staging, (size_t)w.gguf_bytes);
    if (e == hipSuccess) e = hipMemcpyAsync(staging, gguf, (size_t)w.gguf_bytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemsetAsync(g_ctx.dcount, 0, sizeof(unsigned), s);
    if (e == hipSuccess) {
        launch_layout_repack((const uint8_t*)staging, blocks, L, planes, s);
        launch_layout_verify((const uint8_t*)staging, blocks, L, planes, g_ctx.dcount, s);
        e = hipGetLastError();
    }
    unsigned bad = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&bad, g_ctx.dcount, sizeof(unsigned), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (staging) hipFree(staging);
    int rc = OK;
    if (e != hipSuccess) rc = set_error(ERR_DEVICE, std::string("weight_upload: ") + hipGetErrorString(e));
    else if (bad) rc = set_error(ERR_DEVICE, "weight_upload: layout verify found " + std::to_string(bad) + " differing bytes");
    if (rc != OK) {
        hipFree(w.alloc);
        return rc;
    }
    out = w;
    return OK;
}

// Uploads, repacks and byte-verifies one GGUF tensor into w. bank = true lifts
// the per-tensor row limit of llm.rs:248 (expert banks stack many tensors).
int upload_weight(uint32_t kind, int64_t n, int64_t m, const void* gguf, size_t bytes, Weight& out, bool bank) {
    if (int rc = require_ctx()) return rc;
    if (!gguf) return set_error(ERR_ARG, "weight_upload: null pointer");
    FrontierLayout fl;
    const bool split = kind != KIND_Q8_0 && frontier_layout(kind, fl);
    if (kind != KIND_Q8_0 && kind != KIND_Q4_K && kind != KIND_Q3_K && !split)
        return set_error(ERR_QUANT_TYPE, "weight_upload: unsupported kind");
    const int64_t rb = uq::row_bytes(kind, n);
    if (rb < 0 || m <= 0 || n > MAX_N || (!bank && m > MAX_M) || m > (int64_t)1 << 26)
        return set_error(ERR_SHAPE, "weight_upload: bad shape");
    if ((kind == KIND_F32 || kind == KIND_BF16) && n % 8)
        return set_error(ERR_SHAPE, "weight_upload: F32/BF16 rows must hold a multiple of 8 values");
    if ((int64_t)bytes != rb * m) return set_error(ERR_SHAPE, "weight_upload: byte count != rows * row_bytes");
    if (split) return upload_split(kind, n, m, gguf, rb, fl, out);
    hipStream_t s = g_ctx.stream;
    Weight w;
    w.kind = kind;
    w.n = n;
    w.m = m;
    w.gguf_bytes = rb * m;
    size_t total = 0;
    size_t off_q = 0, off_d = 0, off_sc = 0;
    // lm_head-sized Q3_K weights (row blocks for eight workgroups per CU)
    // take the row-block layout; expert banks keep the unit planes that the
    // MoE kernels address by expert row
    SbGeom sg;
    if (kind == KIND_Q3_K && !bank) {
        sg = sb_geom(n, m);
        if (!sg.LB || sg.blocks < 8 * (int64_t)cu_count()) sg = SbGeom();
    }
    if (sg.LB) {
        w.sb_lb = sg.LB;
        w.sb_rb = sg.RB;
        total = align256((size_t)sg.blocks * sg.LB * Q3KSB::P * 16);
    } else if (kind == KIND_Q8_0) {
        off_q = 0;
        off_d = align256((size_t)(n * m));
        total = off_d + align256((size_t)(n / 32 * m) * 2);
    } else if (kind == KIND_Q4_K) {
        const size_t blocks = (size_t)(n / 256 * m);
        off_q = 0;
        off_sc = align256(blocks * 128);
        off_d = off_sc + align256(blocks * 16);
        total = off_d + align256(blocks * 4);
    } else {
        // Q3_K: per superblock four units of 16 + 16 bytes (d inside the second)
        const size_t blocks = (size_t)(n / 256 * m);
        off_q = 0;
        off_sc = align256(blocks * 64);
        off_d = off_sc;
        total = off_sc + align256(blocks * 64);
    }
    UQ_CHECK_HIP(hipMalloc(&w.alloc, total));
    w.alloc_bytes = total;
    uint8_t* base = (uint8_t*)w.alloc;
    w.qs = (const int8_t*)(base + off_q);
    if (!sg.LB) {
        w.d = (const uint16_t*)(base + off_d);
        if (kind != KIND_Q8_0) w.sc = base + off_sc;
    }
    int rc = OK;
    {
        void* staging = nullptr;
        hipError_t e = hipMalloc(&staging, (size_t)w.gguf_bytes);
        if (e == hipSuccess) e = hipMemcpyAsync(staging, gguf, (size_t)w.gguf_bytes, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipMemsetAsync(g_ctx.dcount, 0, sizeof(unsigned), s);
        if (e == hipSuccess && sg.LB) e = hipMemsetAsync(w.alloc, 0, total, s);  // the padding slots
        if (e == hipSuccess) {
            if (sg.LB) {
                launch_sb_repack(kind, (const uint8_t*)staging, n, m, sg.LB, sg.RB, (uint8_t*)w.alloc, g_ctx.dcount, s);
            } else if (kind == KIND_Q8_0) {
                launch_q8_repack((const uint8_t*)staging, m, n / 32, (int8_t*)w.qs, (uint16_t*)w.d, s);
                launch_q8_verify(w.qs, w.d, (const uint8_t*)staging, m, n / 32, g_ctx.dcount, s);
            } else if (kind == KIND_Q4_K) {
                const int64_t blocks = n / 256 * m;
                launch_q4k_repack((const uint8_t*)staging, blocks, n / 256, (int8_t*)w.qs, (uint8_t*)w.sc, (uint32_t*)w.d,
                                  s);
                launch_q4k_verify(w.qs, w.sc, (const uint32_t*)w.d, (const uint8_t*)staging, blocks, n / 256,
                                  g_ctx.dcount, s);
            } else {
                const int64_t blocks = n / 256 * m;
                launch_q3k_repack((const uint8_t*)staging, blocks, (int8_t*)w.qs, (int8_t*)w.sc, (uint16_t*)w.d, s);
                launch_q3k_verify(w.qs, (const int8_t*)w.sc, w.d, (const uint8_t*)staging, blocks, g_ctx.dcount, s);
            }
            e = hipGetLastError();
        }
        unsigned bad = 0;
        if (e == hipSuccess) e = hipMemcpyAsync(&bad, g_ctx.dcount, sizeof(unsigned), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (staging) hipFree(staging);
        if (e != hipSuccess) rc = set_error(ERR_DEVICE, std::string("weight_upload: ") + hipGetErrorString(e));
        else if (bad) rc = set_error(ERR_DEVICE, "weight_upload: repack verify found " + std::to_string(bad) + " differing bytes");
    }
    if (rc != OK) {
        hipFree(w.alloc);
        return rc;
    }
    out = w;
    return OK;
}
}  // namespace uq

extern "C" {

int uq_weight_upload(uint32_t kind, int64_t n, int64_t m, const void* gguf, size_t bytes, uq_weight_t* out) {
    if (!out) return set_error(ERR_ARG, "weight_upload: null pointer");
    Weight w;
    if (int rc = upload_weight(kind, n, m, gguf, bytes, w, false)) return rc;
    *out = new uq_weight{w};
    return OK;
}

int uq_weight_free(uq_weight_t w) {
    if (!w) return OK;
    hipStreamSynchronize(g_ctx.stream);
    hipFree(w->w.alloc);
    delete w;
    return OK;
}

int64_t uq_weight_bytes(uq_weight_t w) { return w ? (int64_t)w->w.alloc_bytes : ERR_ARG; }

static int check_x(const float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++)
        if (!std::isfinite(x[i])) return set_error(ERR_NONFINITE, "input contains a non-finite value");
    return OK;
}

int uq_quant_act_dev(const float* x, int64_t n, int8_t* xq, float* xs, void* stream) {
    if (int rc = require_ctx()) return rc;
    if (!x || !xq || !xs) return set_error(ERR_ARG, "quant_act_dev: null pointer");
    if (n <= 0 || n % 32) return set_error(ERR_SHAPE, "quant_act_dev: n must be a positive multiple of 32");
    launch_quant_act(x, n, xq, xs, pick(stream));
    UQ_CHECK_HIP(hipGetLastError());
    return OK;
}

int uq_matvec_q_dev(uq_weight_t w, const int8_t* xq, const float* xs, float* y, void* stream) {
    if (int rc = require_ctx()) return rc;
    if (!w || !xq || !xs || !y) return set_error(ERR_ARG, "matvec_q_dev: null pointer");
    if (int rc = launch_matvec(w->w, nullptr, xq, xs, y, pick(stream))) return rc;
    UQ_CHECK_HIP(hipGetLastError());
    return OK;
}

int uq_matvec_static(uq_weight_t w, const float* x, float* y, void* stream) {
    if (int rc = require_ctx()) return rc;
    if (!w || !x || !y) return set_error(ERR_ARG, "matvec_static: null pointer");
    const Weight& W = w->w;
    if (W.kind != KIND_Q8_0 && W.kind != KIND_Q4_K && W.kind != KIND_Q3_K)
        return set_error(ERR_QUANT_TYPE, "matvec_static: Q8_0, Q4_K or Q3_K weights only");
    if (W.n > UQ_STATIC_MAX_N)
        return set_error(ERR_SHAPE, "matvec_static: n exceeds the static scratch (16384 values)");
    void* const p = g_ctx.device < MAX_DEVICES ? g_scratch[g_ctx.device] : nullptr;
    if (!p) return set_error(ERR_DEVICE, "matvec_static: no static scratch on this device");
    int8_t* const xq = (int8_t*)p;
    float* const xs = (float*)((int8_t*)p + UQ_STATIC_MAX_N);
    const hipStream_t s = pick(stream);
    // every code and scale the matvec reads is written by this quantization
    // first, so the scratch needs no clearing
    launch_quant_act(x, W.n, xq, xs, s);
    UQ_CHECK_HIP(hipGetLastError());
    if (int rc = launch_matvec(W, nullptr, xq, xs, y, s)) return rc;
    UQ_CHECK_HIP(hipGetLastError());
    return OK;
}

int uq_matvec_table_dev(const uq_weight_t* ws, const uq_weight_t* w2s, int count, const int8_t* xq, const float* xs,
                        float* const* ys, void* stream) {
    if (int rc = require_ctx()) return rc;
    if (!ws || !xq || !xs || !ys || count < 1 || count > 8) return set_error(ERR_ARG, "matvec_table_dev: 1..8 weights");
    const Weight* wl[8];
    const Weight* w2l[8];
    for (int i = 0; i < count; i++) {
        if (!ws[i] || !ys[i]) return set_error(ERR_ARG, "matvec_table_dev: null weight or output");
        wl[i] = &ws[i]->w;
        w2l[i] = w2s && w2s[i] ? &w2s[i]->w : nullptr;
    }
    if (int rc = launch_matvec_multi(wl, w2l, ys, count, xq, xs, pick(stream))) return rc;
    UQ_CHECK_HIP(hipGetLastError());
    return OK;
}

int uq_gateup_q_dev(uq_weight_t gate, uq_weight_t up, const int8_t* xq, const float* xs, float* out, void* stream) {
    if (int rc = require_ctx()) return rc;
    if (!gate || !up || !xq || !xs || !out) return set_error(ERR_ARG, "gateup_q_dev: null pointer");
    if (int rc = launch_matvec(gate->w, &up->w, xq, xs, out, pick(stream))) return rc;
    UQ_CHECK_HIP(hipGetLastError());
    return OK;
}

int uq_batch(const uq_weight_t* ws, int count, const float* x, int64_t n, float* const* ys, const int64_t* ms) {
    if (int rc = require_ctx()) return rc;
    if (!ws || !x || !ys || !ms || count < 1 || count > 3) return set_error(ERR_SHAPE, "batch: 1..3 tensors");
    int64_t total = 0;
    for (int i = 0; i < count; i++) {
        if (!ws[i] || !ys[i]) return set_error(ERR_ARG, "batch: null tensor or output");
        if (ws[i]->w.n != n || ws[i]->w.m != ms[i]) return set_error(ERR_SHAPE, "batch: tensor shape != x/y lengths");
        total += ms[i];
    }
    if (n > MAX_N) return set_error(ERR_SHAPE, "batch: n > 16384");
    if (int rc = check_x(x, n)) return rc;
    if (int rc = ensure_y((size_t)total)) return rc;
    hipStream_t s = g_ctx.stream;
    UQ_CHECK_HIP(hipMemcpyAsync(g_ctx.dx, x, sizeof(float) * n, hipMemcpyHostToDevice, s));
    launch_quant_act(g_ctx.dx, n, g_ctx.dxq, g_ctx.dxs, s);
    int64_t off = 0;
    bool q8 = true;
    for (int i = 0; i < count; i++) q8 = q8 && ws[i]->w.kind == KIND_Q8_0;
    if (q8 && count > 1) {
        // one launch for the batch (the reference's QKV job batch)
        const Weight* wl[3];
        float* yl[3];
        for (int i = 0; i < count; i++) {
            wl[i] = &ws[i]->w;
            yl[i] = g_ctx.dy + off;
            off += ms[i];
        }
        if (int rc = launch_matvec_multi(wl, nullptr, yl, count, g_ctx.dxq, g_ctx.dxs, s)) return rc;
    } else {
        for (int i = 0; i < count; i++) {
            if (int rc = launch_matvec(ws[i]->w, nullptr, g_ctx.dxq, g_ctx.dxs, g_ctx.dy + off, s)) return rc;
            off += ms[i];
        }
    }
    UQ_CHECK_HIP(hipGetLastError());
    std::vector<float> host((size_t)total);
    UQ_CHECK_HIP(hipMemcpyAsync(host.data(), g_ctx.dy, sizeof(float) * total, hipMemcpyDeviceToHost, s));
    UQ_CHECK_HIP(hipStreamSynchronize(s));
    off = 0;
    for (int i = 0; i < count; i++) {
        std::memcpy(ys[i], host.data() + off, sizeof(float) * ms[i]);
        off += ms[i];
    }
    if (int rc = check_x(host.data(), total)) return set_error(rc, "batch: non-finite output");
    return OK;
}

int uq_matvec(uq_weight_t w, const float* x, int64_t n, float* y, int64_t m) {
    float* ys[1] = {y};
    int64_t ms[1] = {m};
    return uq_batch(&w, 1, x, n, ys, ms);
}

int uq_quant_act(const float* x, int64_t n, int8_t* q, float* scale) {
    if (int rc = require_ctx()) return rc;
    if (!x || !q || !scale) return set_error(ERR_ARG, "quant_act: null pointer");
    if (n <= 0 || n % 32 || n > MAX_N) return set_error(ERR_SHAPE, "quant_act: n must be a multiple of 32, <= 16384");
    hipStream_t s = g_ctx.stream;
    UQ_CHECK_HIP(hipMemcpyAsync(g_ctx.dx, x, sizeof(float) * n, hipMemcpyHostToDevice, s));
    launch_quant_act(g_ctx.dx, n, g_ctx.dxq, g_ctx.dxs, s);
    UQ_CHECK_HIP(hipGetLastError());
    UQ_CHECK_HIP(hipMemcpyAsync(q, g_ctx.dxq, n, hipMemcpyDeviceToHost, s));
    UQ_CHECK_HIP(hipMemcpyAsync(scale, g_ctx.dxs, sizeof(float) * (n / 32), hipMemcpyDeviceToHost, s));
    UQ_CHECK_HIP(hipStreamSynchronize(s));
    return OK;
}

int uq_block_dots(uq_weight_t w, const float* x, int64_t n, int32_t* dots, int64_t count) {
    if (int rc = require_ctx()) return rc;
    if (!w || !x || !dots) return set_error(ERR_ARG, "block_dots: null pointer");
    if (w->w.n != n) return set_error(ERR_SHAPE, "block_dots: x length != tensor n");
    const int bsz = w->w.kind == KIND_Q3_K ? 16 : 32;
    if (count != w->w.m * (n / bsz)) return set_error(ERR_SHAPE, "block_dots: wrong output count");
    hipStream_t s = g_ctx.stream;
    int32_t* d = nullptr;
    UQ_CHECK_HIP(hipMalloc(&d, sizeof(int32_t) * count));
    int rc = OK;
    hipError_t e = hipMemcpyAsync(g_ctx.dx, x, sizeof(float) * n, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) {
        launch_quant_act(g_ctx.dx, n, g_ctx.dxq, g_ctx.dxs, s);
        rc = launch_block_dots(w->w, g_ctx.dxq, d, s);
        e = hipGetLastError();
    }
    if (e == hipSuccess && rc == OK) e = hipMemcpyAsync(dots, d, sizeof(int32_t) * count, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    hipFree(d);
    if (e != hipSuccess) return set_error(ERR_DEVICE, std::string("block_dots: ") + hipGetErrorString(e));
    return rc;
}

int uq_dev_alloc(size_t bytes, void** ptr) {
    if (int rc = require_ctx()) return rc;
    if (!ptr) return set_error(ERR_ARG, "dev_alloc: null pointer");
    UQ_CHECK_HIP(hipMalloc(ptr, bytes ? bytes : 1));
    return OK;
}
int uq_dev_free(void* ptr) {
    if (ptr) {
        hipStreamSynchronize(g_ctx.stream);
        UQ_CHECK_HIP(hipFree(ptr));
    }
    return OK;
}
int uq_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    if (int rc = require_ctx()) return rc;
    UQ_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_ctx.stream));
    UQ_CHECK_HIP(hipStreamSynchronize(g_ctx.stream));
    return OK;
}
int uq_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (int rc = require_ctx()) return rc;
    UQ_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_ctx.stream));
    UQ_CHECK_HIP(hipStreamSynchronize(g_ctx.stream));
    return OK;
}

int uq_time_matvecs(const uq_weight_t* ws, const int* pairs, int count, int64_t max_n, int reps, int warmup,
                    int probe, double* total_ms, double* probe_ms) {
    if (int rc = require_ctx()) return rc;
    if (!ws || count <= 0 || reps <= 0 || warmup < 0 || !total_ms) return set_error(ERR_ARG, "time_matvecs: bad args");
    hipStream_t s = g_ctx.stream;
    int64_t ymax = 0;
    for (int i = 0; i < count; i++) {
        if (!ws[i]) return set_error(ERR_ARG, "time_matvecs: null weight");
        if (ws[i]->w.n > max_n) return set_error(ERR_SHAPE, "time_matvecs: weight n > max_n");
        if (ws[i]->w.m > ymax) ymax = ws[i]->w.m;
    }
    // a seeded-constant activation: 0.5 everywhere except a ramp, quantized once
    std::vector<float> hx((size_t)max_n);
    for (int64_t i = 0; i < max_n; i++) hx[i] = (float)((i * 37) % 251) / 125.0f - 1.0f;
    float *x = nullptr, *y = nullptr, *xs = nullptr;
    int8_t* xq = nullptr;
    UQ_CHECK_HIP(hipMalloc(&x, sizeof(float) * max_n));
    UQ_CHECK_HIP(hipMalloc(&xq, max_n));
    UQ_CHECK_HIP(hipMalloc(&xs, sizeof(float) * (max_n / 32)));
    UQ_CHECK_HIP(hipMalloc(&y, sizeof(float) * ymax));
    UQ_CHECK_HIP(hipMemcpyAsync(x, hx.data(), sizeof(float) * max_n, hipMemcpyHostToDevice, s));
    launch_quant_act(x, max_n, xq, xs, s);
    std::vector<hipEvent_t> pev;
    hipEvent_t t0, t1;
    UQ_CHECK_HIP(hipEventCreate(&t0));
    UQ_CHECK_HIP(hipEventCreate(&t1));
    const int nprobe = probe >= 0 ? reps : 0;
    pev.resize(2 * (size_t)nprobe);
    for (auto& e : pev) UQ_CHECK_HIP(hipEventCreate(&e));
    int rc = OK;
    for (int r = 0; r < warmup + reps && rc == OK; r++) {
        const bool timed = r >= warmup;
        if (r == warmup) UQ_CHECK_HIP(hipEventRecord(t0, s));
        for (int i = 0; i < count && rc == OK; i++) {
            const bool pair = pairs && pairs[i] && i + 1 < count;
            const bool rec = timed && i == probe;
            if (rec) UQ_CHECK_HIP(hipEventRecord(pev[2 * (r - warmup)], s));
            rc = launch_matvec(ws[i]->w, pair ? &ws[i + 1]->w : nullptr, xq, xs, y, s);
            if (rec) UQ_CHECK_HIP(hipEventRecord(pev[2 * (r - warmup) + 1], s));
            if (pair) i++;
        }
    }
    UQ_CHECK_HIP(hipEventRecord(t1, s));
    UQ_CHECK_HIP(hipEventSynchronize(t1));
    float ms = 0;
    UQ_CHECK_HIP(hipEventElapsedTime(&ms, t0, t1));
    *total_ms = ms;
    if (probe_ms) {
        double sum = 0;
        for (int r = 0; r < nprobe; r++) {
            float p = 0;
            UQ_CHECK_HIP(hipEventElapsedTime(&p, pev[2 * r], pev[2 * r + 1]));
            sum += p;
        }
        *probe_ms = nprobe ? sum / nprobe : 0.0;
    }
    for (auto& e : pev) hipEventDestroy(e);
    hipEventDestroy(t0);
    hipEventDestroy(t1);
    hipFree(x);
    hipFree(xq);
    hipFree(xs);
    hipFree(y);
    return rc;
}

int uq_time_matvec_tables(const uq_weight_t* ws, const int* pairs, int count, int64_t max_n, int reps, int warmup,
                          double* total_ms) {
    if (int rc = require_ctx()) return rc;
    if (!ws || count <= 0 || reps <= 0 || warmup < 0 || !total_ms) return set_error(ERR_ARG, "time_matvec_tables: bad args");
    hipStream_t s = g_ctx.stream;
    int64_t ysum = 0;
    for (int i = 0; i < count; i++) {
        if (!ws[i]) return set_error(ERR_ARG, "time_matvec_tables: null weight");
        if (ws[i]->w.n > max_n) return set_error(ERR_SHAPE, "time_matvec_tables: weight n > max_n");
        ysum += ws[i]->w.m;
    }
    // consecutive weights of one input length form one table; pairs[i] marks a gate/up pair (i, i+1)
    struct Table { std::vector<const Weight*> w, w2; std::vector<float*> y; };
    std::vector<Table> tables;
    float *x = nullptr, *y = nullptr, *xs = nullptr;
    int8_t* xq = nullptr;
    UQ_CHECK_HIP(hipMalloc(&x, sizeof(float) * max_n));
    UQ_CHECK_HIP(hipMalloc(&xq, max_n));
    UQ_CHECK_HIP(hipMalloc(&xs, sizeof(float) * (max_n / 32)));
    UQ_CHECK_HIP(hipMalloc(&y, sizeof(float) * ysum));
    std::vector<float> hx((size_t)max_n);
    for (int64_t i = 0; i < max_n; i++) hx[i] = (float)((i * 37) % 251) / 125.0f - 1.0f;
    UQ_CHECK_HIP(hipMemcpyAsync(x, hx.data(), sizeof(float) * max_n, hipMemcpyHostToDevice, s));
    launch_quant_act(x, max_n, xq, xs, s);
    int64_t yo = 0;
    for (int i = 0; i < count; i++) {
        const bool pair = pairs && pairs[i] && i + 1 < count;
        if (tables.empty() || tables.back().w.back()->n != ws[i]->w.n || tables.back().w.size() == 8) tables.emplace_back();
        tables.back().w.push_back(&ws[i]->w);
        tables.back().w2.push_back(pair ? &ws[i + 1]->w : nullptr);
        tables.back().y.push_back(y + yo);
        yo += ws[i]->w.m;
        if (pair) i++;
    }
    hipEvent_t t0, t1;
    UQ_CHECK_HIP(hipEventCreate(&t0));
    UQ_CHECK_HIP(hipEventCreate(&t1));
    int rc = OK;
    for (int r = 0; r < warmup + reps && rc == OK; r++) {
        if (r == warmup) UQ_CHECK_HIP(hipEventRecord(t0, s));
        for (const Table& t : tables) {
            rc = launch_matvec_multi(t.w.data(), t.w2.data(), t.y.data(), (int)t.w.size(), xq, xs, s);
            if (rc) break;
        }
    }
    UQ_CHECK_HIP(hipEventRecord(t1, s));
    UQ_CHECK_HIP(hipEventSynchronize(t1));
    float ms = 0;
    UQ_CHECK_HIP(hipEventElapsedTime(&ms, t0, t1));
    hipEventDestroy(t0);
    hipEventDestroy(t1);
    hipFree(x);
    hipFree(xq);
    hipFree(xs);
    hipFree(y);
    if (rc) return rc;
    *total_ms = ms;
    return OK;
}

}  // extern "C"
