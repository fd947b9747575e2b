"""Python binding of libuq.so (the C ABI declared in include/uq.h).

A thin ctypes layer for tests and the benchmark, plus host-side helpers that
mirror the reference runtime's call surface (driver/src/llm.rs:63 ``Tensor``,
:226 ``Gpu::batch``, :246 ``Gpu::matvec``; frontier_forward.rs:10 ``Error``).

The library must be built (``python uefi-gpu_amd/build_lib.py`` or
``__graft_entry__.build()``); importing this module never falls back to any
CPU path: a missing library raises ``UqError``.
"""
import ctypes
import enum
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libuq.so")

OK = 0
KIND_F32, KIND_Q8_0, KIND_Q3_K, KIND_Q4_K = 0, 8, 11, 12
KIND_Q6_K, KIND_IQ3_XXS, KIND_IQ4_NL, KIND_IQ4_XS, KIND_BF16 = 14, 18, 20, 23, 30
# kinds of the fp32-activation reader (frontier_core.rs:53-58)
LINEAR_KINDS = (KIND_F32, KIND_BF16, KIND_Q8_0, KIND_Q6_K, KIND_IQ3_XXS, KIND_IQ4_NL, KIND_IQ4_XS)


class Error(enum.IntEnum):
    """Status codes (frontier_forward.rs:10 Error, frontier_core.rs:37 QuantType)."""
    SHAPE = -1
    QUANT_TYPE = -2
    NONFINITE = -3
    DEVICE = -4
    TIMEOUT = -5
    CONTEXT = -6
    ARG = -7
    FORMAT = -8


class UqError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__("%s: %s" % (Error(status).name if status in Error._value2member_map_ else status, msg))
        self.status = status


_lib = None

_c_f32p = ctypes.POINTER(ctypes.c_float)
_c_i8p = ctypes.POINTER(ctypes.c_int8)
_c_i32p = ctypes.POINTER(ctypes.c_int32)
_c_u8p = ctypes.POINTER(ctypes.c_uint8)
_c_u32p = ctypes.POINTER(ctypes.c_uint32)
_c_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64

# name -> (restype, argtypes)
_SIGS = {
    "uq_init": (ctypes.c_int, [ctypes.c_int]),
    "uq_shutdown": (ctypes.c_int, []),
    "uq_last_error": (ctypes.c_char_p, []),
    "uq_stream": (_vp, []),
    "uq_sync": (ctypes.c_int, []),
    "uq_row_bytes": (_i64, [ctypes.c_uint32, _i64]),
    "uq_weight_upload": (ctypes.c_int, [ctypes.c_uint32, _i64, _i64, _vp, ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "uq_weight_free": (ctypes.c_int, [_vp]),
    "uq_weight_bytes": (_i64, [_vp]),
    "uq_matvec": (ctypes.c_int, [_vp, _c_f32p, _i64, _c_f32p, _i64]),
    "uq_batch": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.c_int, _c_f32p, _i64, ctypes.POINTER(_c_f32p), _c_i64p]),
    "uq_quant_act_dev": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp]),
    "uq_matvec_q_dev": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "uq_matvec_static": (ctypes.c_int, [_vp, _vp, _vp, _vp]),
    "uq_gateup_q_dev": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "uq_matvec_table_dev": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.c_int, _vp, _vp,
                                           ctypes.POINTER(_vp), _vp]),
    "uq_quant_act": (ctypes.c_int, [_c_f32p, _i64, _c_i8p, _c_f32p]),
    "uq_block_dots": (ctypes.c_int, [_vp, _c_f32p, _i64, _c_i32p, _i64]),
    "uq_dequantize": (ctypes.c_int, [ctypes.c_uint32, _vp, ctypes.c_size_t, _i64, _c_f32p]),
    "uq_linear": (ctypes.c_int, [_vp, _c_f32p, _i64, _c_f32p, _i64]),
    "uq_linear_batch": (ctypes.c_int, [_vp, ctypes.c_int]),
    "uq_linear_dev": (ctypes.c_int, [_vp, _vp, _vp, _vp]),
    "uq_linear_multi_dev": (ctypes.c_int, [_vp, ctypes.c_int, _vp]),
    "uq_time_linear_tables": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int,
                                             ctypes.POINTER(ctypes.c_double)]),
    "uq_time_linear": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.POINTER(ctypes.c_double)]),
    "uq_dev_alloc": (ctypes.c_int, [ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "uq_dev_free": (ctypes.c_int, [_vp]),
    "uq_memcpy_h2d": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t]),
    "uq_memcpy_d2h": (ctypes.c_int, [_vp, _vp, ctypes.c_size_t]),
    "uq_time_matvec_tables": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.POINTER(ctypes.c_int), ctypes.c_int, _i64,
                                             ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]),
    "uq_time_matvecs": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.POINTER(ctypes.c_int), ctypes.c_int, _i64,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "uq_model_create": (ctypes.c_int, [_vp, ctypes.POINTER(_vp)]),
    "uq_model_free": (ctypes.c_int, [_vp]),
    "uq_model_set_tensor": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_uint32, _i64, _i64, _vp, ctypes.c_size_t]),
    "uq_model_prepare": (ctypes.c_int, [_vp]),
    "uq_decode_step": (ctypes.c_int, [_vp, ctypes.c_uint32, ctypes.c_int, _c_u32p]),
    "uq_decode_run": (ctypes.c_int, [_vp, ctypes.c_uint32, ctypes.c_int, ctypes.c_int, _c_u32p,
                                     ctypes.POINTER(ctypes.c_double)]),
    "uq_model_logits": (ctypes.c_int, [_vp, _c_f32p, _i64]),
    "uq_prefill": (ctypes.c_int, [_vp, _c_u32p, ctypes.c_int, _c_u32p]),
    "uq_prefill_gemm": (ctypes.c_int, [_vp, _c_i8p, _c_f32p, _i64, _c_f32p]),
    "uq_time_prefill_gemm": (ctypes.c_int, [_vp, _vp, _i64, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]),
    "uq_time_prefill_attention": (ctypes.c_int, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                                 ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]),
    "uq_prompt_tokens": (ctypes.c_int, [_vp, _c_u32p, ctypes.c_int, ctypes.c_int, _c_u32p]),
    "uq_probe_bandwidth": (ctypes.c_int, [_i64, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                          ctypes.POINTER(ctypes.c_double)]),
    "uq_probe_mfma": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_double)]),
    "uq_model_kv": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_uint16),
                                   ctypes.POINTER(ctypes.c_uint16)]),
    "uq_moe_create": (ctypes.c_int, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_uint32,
                                     ctypes.POINTER(_vp)]),
    "uq_moe_free": (ctypes.c_int, [_vp]),
    "uq_moe_set_expert": (ctypes.c_int, [_vp, ctypes.c_int32, _vp, _vp, _vp]),
    "uq_moe_set_shared": (ctypes.c_int, [_vp, ctypes.c_uint32, _vp, _vp, _vp, _c_f32p]),
    "uq_moe_ffn": (ctypes.c_int, [_vp, _c_f32p, _c_f32p, _c_f32p, _c_i32p, _c_f32p]),
    "uq_moe_ffn_dev": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "uq_moe_run": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]),
    "uq_gguf_parse": (ctypes.c_int, [_vp, ctypes.c_size_t, ctypes.c_uint64, ctypes.POINTER(_vp),
                                     ctypes.POINTER(ctypes.c_int)]),
    "uq_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_vp), ctypes.POINTER(ctypes.c_int)]),
    "uq_gguf_free": (ctypes.c_int, [_vp]),
    "uq_gguf_tensor_count": (_i64, [_vp]),
    "uq_gguf_data_offset": (ctypes.c_uint64, [_vp]),
    "uq_gguf_split_info": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                                          ctypes.POINTER(ctypes.c_uint64)]),
    "uq_gguf_tensor_info": (ctypes.c_int, [_vp, _i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_uint32),
                                           ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_uint64),
                                           ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "uq_gguf_find_tensor": (_i64, [_vp, ctypes.c_char_p]),
    "uq_gguf_meta_u64": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
    "uq_gguf_meta_f32": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)]),
    "uq_gguf_meta_str": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_vp), ctypes.POINTER(ctypes.c_uint64)]),
    "uq_gguf_meta_array": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32),
                                          ctypes.POINTER(ctypes.c_uint64)]),
    "uq_gguf_qwen2_config": (ctypes.c_int, [_vp, ctypes.c_int32, _vp]),
    "uq_gguf_meta_array_str": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_uint64, ctypes.POINTER(_vp),
                                              ctypes.POINTER(ctypes.c_uint64)]),
    "uq_gguf_tensor_rows": (ctypes.c_int, [_vp, _i64, ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64),
                                           ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_int)]),
    "uq_gguf_tensor_expert": (ctypes.c_int, [_vp, _i64, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint64),
                                             ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_int)]),
    "uq_gguf_index_create": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.c_int, ctypes.POINTER(_vp),
                                            ctypes.POINTER(ctypes.c_int)]),
    "uq_gguf_index_free": (ctypes.c_int, [_vp]),
    "uq_gguf_index_shard_count": (ctypes.c_int, [_vp]),
    "uq_gguf_index_shard": (_vp, [_vp, ctypes.c_int]),
    "uq_gguf_index_find": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_i64),
                                          ctypes.POINTER(ctypes.c_int)]),
    "uq_gguf_index_inventory": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_int)]),
    "uq_gguf_load_weight": (ctypes.c_int, [_vp, _i64, ctypes.c_int32, ctypes.POINTER(_vp)]),
    "uq_moe_load_gguf": (ctypes.c_int, [_vp, _vp, ctypes.c_int32]),
    "uq_moe_info": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
                                   ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
                                   ctypes.POINTER(ctypes.c_uint32)]),
    "uq_device_memory": (ctypes.c_int, [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]),
    "uq_gguf_token_text": (ctypes.c_int, [_vp, ctypes.c_uint32, _vp, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)]),
    "uq_generate": (ctypes.c_int, [_vp, _c_u32p, ctypes.c_int, ctypes.c_int, _c_u32p, ctypes.c_int, _c_u32p,
                                   ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                                   ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "uq_model_load_gguf": (ctypes.c_int, [_vp, _vp]),
    "uq_synth_quant": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint64, _i64, _i64, _c_u8p]),
    "uq_synth_normal": (ctypes.c_int, [ctypes.c_uint64, _i64, ctypes.c_float, ctypes.c_float, _c_f32p]),
    "uq_synth_tokens": (ctypes.c_int, [ctypes.c_uint64, _i64, ctypes.c_uint32, _c_u32p]),
}


def declared_symbols():
    return sorted(_SIGS)


def lib():
    """Load libuq.so (raises UqError if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise UqError(Error.ARG, "libuq.so not built at %s (run __graft_entry__.build())" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(rc):
    if rc != OK:
        raise UqError(rc, lib().uq_last_error().decode(errors="replace"))
    return rc


def _p(a, ct):
    return a.ctypes.data_as(ct)


def init(device=0):
    _check(lib().uq_init(device))


def shutdown():
    _check(lib().uq_shutdown())


def row_bytes(kind, n):
    return int(lib().uq_row_bytes(kind, n))


# ---------------------------------------------------------------- synthetic data
def synth_quant(kind, seed, rows, n):
    out = np.empty(rows * row_bytes(kind, n), dtype=np.uint8)
    _check(lib().uq_synth_quant(kind, seed & (2**64 - 1), rows, n, _p(out, _c_u8p)))
    return out


def synth_normal(seed, n, mean=0.0, std=1.0):
    out = np.empty(n, dtype=np.float32)
    _check(lib().uq_synth_normal(seed & (2**64 - 1), n, mean, std, _p(out, _c_f32p)))
    return out


def synth_tokens(seed, n, vocab):
    out = np.empty(n, dtype=np.uint32)
    _check(lib().uq_synth_tokens(seed & (2**64 - 1), n, vocab, _p(out, _c_u32p)))
    return out


def fnv1a64(text):
    h = 0xCBF29CE484222325
    for b in text.encode():
        h = ((h ^ b) * 0x100000001B3) & (2**64 - 1)
    return h


def tensor_seed(base, name):
    """Per-tensor seed of a synthetic model: base mixed with FNV-1a of the GGUF name."""
    return ((base * 0x9E3779B97F4A7C15) ^ fnv1a64(name)) & (2**64 - 1)


# ---------------------------------------------------------------- weights / linears
class Weight:
    """A device-resident, verified, repacked GGUF tensor (uq_weight_t)."""

    def __init__(self, kind, n, m, gguf_bytes):
        self.kind, self.n, self.m = kind, int(n), int(m)
        buf = np.ascontiguousarray(gguf_bytes, dtype=np.uint8)
        h = _vp()
        _check(lib().uq_weight_upload(kind, self.n, self.m, buf.ctypes.data, buf.nbytes, ctypes.byref(h)))
        self.handle = h

    def free(self):
        if self.handle:
            lib().uq_weight_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @property
    def device_bytes(self):
        return int(lib().uq_weight_bytes(self.handle))


def matvec(w, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(w.m, dtype=np.float32)
    _check(lib().uq_matvec(w.handle, _p(x, _c_f32p), x.size, _p(y, _c_f32p), y.size))
    return y


def batch(ws, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    ys = [np.empty(w.m, dtype=np.float32) for w in ws]
    handles = (_vp * len(ws))(*[w.handle for w in ws])
    yp = (_c_f32p * len(ws))(*[_p(y, _c_f32p) for y in ys])
    ms = (ctypes.c_int64 * len(ws))(*[w.m for w in ws])
    _check(lib().uq_batch(handles, len(ws), _p(x, _c_f32p), x.size, yp, ms))
    return ys


class LinearJob(ctypes.Structure):
    """uq_linear_job: one entry of the FrontierJob table."""
    _fields_ = [("weight", _vp), ("x", _vp), ("y", _vp)]


def dequantize(kind, raw, n):
    """frontier_dequant: the n values of a GGUF byte run as f32 (bit-exact)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(int(n), dtype=np.float32)
    _check(lib().uq_dequantize(kind, raw.ctypes.data, raw.nbytes, int(n), _p(out, _c_f32p)))
    return out


def linear(w, x):
    """Weights::linear over frontier_matvec: y = W x with fp32 x."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(w.m, dtype=np.float32)
    _check(lib().uq_linear(w.handle, _p(x, _c_f32p), x.size, _p(y, _c_f32p), y.size))
    return y


def linear_batch(pairs):
    """Weights::batch: [(weight, x), ...] in one launch; returns the outputs."""
    xs = [np.ascontiguousarray(x, dtype=np.float32) for _, x in pairs]
    ys = [np.empty(w.m, dtype=np.float32) for w, _ in pairs]
    jobs = (LinearJob * len(pairs))(*[LinearJob(w.handle, x.ctypes.data, y.ctypes.data)
                                      for (w, _), x, y in zip(pairs, xs, ys)])
    _check(lib().uq_linear_batch(jobs, len(pairs)))
    return ys


def time_linear(weights, reps, warmup):
    """HIP-event time (ms) of `reps` rounds of one fp32-activation linear per weight."""
    handles = (_vp * len(weights))(*[w.handle for w in weights])
    ms = ctypes.c_double()
    _check(lib().uq_time_linear(handles, len(weights), reps, warmup, ctypes.byref(ms)))
    return ms.value


def quant_act(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.size, dtype=np.int8)
    s = np.empty(x.size // 32, dtype=np.float32)
    _check(lib().uq_quant_act(_p(x, _c_f32p), x.size, _p(q, _c_i8p), _p(s, _c_f32p)))
    return q, s


def block_dots(w, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    bsz = 16 if w.kind == KIND_Q3_K else 32
    d = np.empty(w.m * (w.n // bsz), dtype=np.int32)
    _check(lib().uq_block_dots(w.handle, _p(x, _c_f32p), x.size, _p(d, _c_i32p), d.size))
    return d.reshape(w.m, w.n // bsz)


def prefill_gemm(w, xq, xs):
    """The int8-MFMA prefill GEMM on pre-quantized activations xq [tokens][n], xs [tokens][n/32]."""
    xq = np.ascontiguousarray(xq, np.int8)
    xs = np.ascontiguousarray(xs, np.float32)
    tokens = xq.shape[0]
    y = np.empty((tokens, w.m), np.float32)
    _check(lib().uq_prefill_gemm(w.handle, _p(xq, _c_i8p), _p(xs, _c_f32p), tokens, _p(y, _c_f32p)))
    return y


def time_prefill_gemm(w, w2, tokens, reps):
    ms = ctypes.c_double()
    _check(lib().uq_time_prefill_gemm(w.handle, w2.handle if w2 else None, tokens, reps, ctypes.byref(ms)))
    return ms.value


def time_prefill_attention(tokens, heads, kv_heads, head_dim, quant_out, reps):
    """Mean HIP-event ms of the prefill's causal attention on synthetic q and fp16 K/V."""
    ms = ctypes.c_double()
    _check(lib().uq_time_prefill_attention(tokens, heads, kv_heads, head_dim, 1 if quant_out else 0, reps,
                                           ctypes.byref(ms)))
    return ms.value


def probe_mfma(kind):
    """Achievable matrix-core rate: kind 0 int8 (TOPS), 1 fp16, 2 fp64 (TFLOP/s); one
    wave per SIMD: 3 fp64 MFMAs, 4 with an fp16 operand conversion per MFMA, 5 the
    conversions alone; 6 int8 MFMAs, 7 beside the per-block f32 rescale, 8 the
    rescale alone (rates of the same MFMA count); 16 waves per CU: 9 the int8
    32x32x32 form, 10 the int8 16x16x64 form (TOPS)."""
    t = ctypes.c_double()
    _check(lib().uq_probe_mfma(kind, ctypes.byref(t)))
    return t.value


def probe_bandwidth(nbytes=1 << 30, reps=10):
    r, c = ctypes.c_double(), ctypes.c_double()
    _check(lib().uq_probe_bandwidth(nbytes, reps, ctypes.byref(r), ctypes.byref(c)))
    return r.value, c.value


def time_matvec_tables(weights, pairs, max_n, reps, warmup):
    """HIP-event ms of `reps` rounds, consecutive same-K weights as one job-table launch."""
    handles = (_vp * len(weights))(*[w.handle for w in weights])
    pr = (ctypes.c_int * len(weights))(*pairs)
    ms = ctypes.c_double()
    _check(lib().uq_time_matvec_tables(handles, pr, len(weights), max_n, reps, warmup, ctypes.byref(ms)))
    return ms.value


def time_matvecs(weights, pairs, max_n, reps, warmup, probe):
    hs = (_vp * len(weights))(*[w.handle for w in weights])
    pr = (ctypes.c_int * len(weights))(*pairs)
    tot, pm = ctypes.c_double(), ctypes.c_double()
    _check(lib().uq_time_matvecs(hs, pr, len(weights), max_n, reps, warmup, probe, ctypes.byref(tot), ctypes.byref(pm)))
    return tot.value, pm.value


# ---------------------------------------------------------------- reference-shaped host API
class Tensor:
    """Tensor{name, n, m, typ, off} of driver/src/llm.rs:63 (n = columns, m = rows)."""

    def __init__(self, name, n, m, typ, data):
        self.name, self.n, self.m, self.typ, self.data = name, n, m, typ, data


class Gpu:
    """The reference's linear call surface (llm.rs:226-273) over libuq.

    ``matvec``/``batch`` run matvec_q8 on fp32 x (llm.rs:294-297; the jobs of
    ``batch`` copy that launch, llm.rs:202-214), so they map to the
    fp32-activation reader, ``uq_linear_batch`` with Q8_0 weights. They return
    False on any failure, as the reference does, including its shape rule
    (llm.rs:248); ``last_error`` keeps the message.
    """

    def __init__(self, device=0):
        init(device)
        self.weights = {}
        self.last_error = ""

    def upload(self, t):
        self.weights[t.name] = Weight(t.typ, t.n, t.m, t.data)

    def matvec(self, t, x, y):
        return self.batch([t], x, [y])

    def batch(self, tensors, x, ys):
        if len(tensors) != len(ys) or not 1 <= len(tensors) <= 3:
            return False
        try:
            for t, y in zip(tensors, ys):
                if (t.typ != KIND_Q8_0 or t.n != len(x) or t.m != len(y) or t.n % 32 or t.n > 16384
                        or t.m > 160000):
                    return False
            x = np.ascontiguousarray(x, dtype=np.float32)
            outs = linear_batch([(self.weights[t.name], x) for t in tensors])
        except (UqError, KeyError) as e:
            self.last_error = str(e)
            return False
        for y, o in zip(ys, outs):
            y[:] = o
        return True


# ---------------------------------------------------------------- Qwen2 dense decoder
class Qwen2Config(ctypes.Structure):
    """uq_qwen2_config: the shape constants of driver/src/llm.rs:314-321."""
    _fields_ = [(n, ctypes.c_int32) for n in ("layers", "dim", "hidden", "heads", "kv_heads", "head_dim",
                                             "vocab", "max_seq")] + [("eps", ctypes.c_float), ("theta", ctypes.c_float)]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


QWEN25_15B = dict(layers=28, dim=1536, hidden=8960, heads=12, kv_heads=2, head_dim=128, vocab=151936,
                  max_seq=1024, eps=1e-6, theta=1e6)


def synth_qwen2(cfg, seed):
    """Seeded random-init Qwen2 tensors in GGUF layout: name -> (kind, n, rows, array).
    Q8_0 matrices from uq_synth_quant; norm weights 1 + 0.1 N(0,1); biases 0.02 N(0,1)."""
    D, H, kvd = cfg["dim"], cfg["hidden"], cfg["kv_heads"] * cfg["head_dim"]
    t = {}

    def q8(name, n, rows):
        t[name] = (KIND_Q8_0, n, rows, synth_quant(KIND_Q8_0, tensor_seed(seed, name), rows, n))

    def f32(name, n, mean, std):
        t[name] = (KIND_F32, n, 1, synth_normal(tensor_seed(seed, name), n, mean, std))

    q8("token_embd.weight", D, cfg["vocab"])
    q8("output.weight", D, cfg["vocab"])
    f32("output_norm.weight", D, 1.0, 0.1)
    for l in range(cfg["layers"]):
        b = "blk.%d." % l
        q8(b + "attn_q.weight", D, D)
        q8(b + "attn_k.weight", D, kvd)
        q8(b + "attn_v.weight", D, kvd)
        q8(b + "attn_output.weight", D, D)
        q8(b + "ffn_gate.weight", D, H)
        q8(b + "ffn_up.weight", D, H)
        q8(b + "ffn_down.weight", H, D)
        f32(b + "attn_norm.weight", D, 1.0, 0.1)
        f32(b + "ffn_norm.weight", D, 1.0, 0.1)
        f32(b + "attn_q.bias", D, 0.0, 0.02)
        f32(b + "attn_k.bias", kvd, 0.0, 0.02)
        f32(b + "attn_v.bias", kvd, 0.0, 0.02)
    return t


class Qwen2Model:
    """The decode graph of driver/src/gpu_graph.rs over libuq (uq_model_*)."""

    def __init__(self, cfg, tensors=None):
        self.cfg = dict(cfg)
        c = Qwen2Config(**self.cfg)
        h = _vp()
        _check(lib().uq_model_create(ctypes.byref(c), ctypes.byref(h)))
        self.handle = h
        if tensors:
            for name, (kind, n, rows, arr) in tensors.items():
                self.set_tensor(name, kind, n, rows, arr)
            self.prepare()

    @classmethod
    def from_gguf(cls, path, max_seq=0):
        """A model with the shape constants and tensors of a Qwen2 GGUF file
        (uq_gguf_qwen2_config + uq_model_load_gguf), prepared."""
        g = Gguf.open(path)
        try:
            m = cls(g.qwen2_config(max_seq))
            _check(lib().uq_model_load_gguf(m.handle, g.handle))
            m.prepare()
        finally:
            g.free()
        return m

    def set_tensor(self, name, kind, n, rows, arr):
        a = np.ascontiguousarray(arr)
        _check(lib().uq_model_set_tensor(self.handle, name.encode(), kind, n, rows, a.ctypes.data, a.nbytes))

    def prepare(self):
        _check(lib().uq_model_prepare(self.handle))

    def decode_step(self, token, pos):
        nxt = ctypes.c_uint32()
        _check(lib().uq_decode_step(self.handle, token, pos, ctypes.byref(nxt)))
        return nxt.value

    def decode_run(self, token, pos, steps):
        out = np.empty(steps, np.uint32)
        ms = ctypes.c_double()
        _check(lib().uq_decode_run(self.handle, token, pos, steps, _p(out, _c_u32p), ctypes.byref(ms)))
        return out, ms.value

    def prefill(self, tokens):
        t = np.ascontiguousarray(tokens, np.uint32)
        nxt = ctypes.c_uint32()
        _check(lib().uq_prefill(self.handle, _p(t, _c_u32p), t.size, ctypes.byref(nxt)))
        return nxt.value

    def generate(self, prompt, max_new, stop=(151645, 151643)):
        """generate_one (llm.rs:402-428): prefill, then greedy steps until a stop
        id or max_new tokens. Returns (ids, ended, prefill_ms, decode_ms)."""
        t = np.ascontiguousarray(prompt, np.uint32)
        st = np.ascontiguousarray(stop, np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n, ended = ctypes.c_int(), ctypes.c_int()
        pms, dms = ctypes.c_double(), ctypes.c_double()
        _check(lib().uq_generate(self.handle, _p(t, _c_u32p), t.size, max_new, _p(st, _c_u32p), st.size,
                                 _p(out, _c_u32p), ctypes.byref(n), ctypes.byref(ended), ctypes.byref(pms),
                                 ctypes.byref(dms)))
        return out[:n.value].copy(), bool(ended.value), pms.value, dms.value

    def prompt(self, tokens, pos=0):
        t = np.ascontiguousarray(tokens, np.uint32)
        nxt = ctypes.c_uint32()
        _check(lib().uq_prompt_tokens(self.handle, _p(t, _c_u32p), t.size, pos, ctypes.byref(nxt)))
        return nxt.value

    def logits(self):
        out = np.empty(self.cfg["vocab"], np.float32)
        _check(lib().uq_model_logits(self.handle, _p(out, _c_f32p), out.size))
        return out

    def kv(self, layer, count):
        kvd = self.cfg["kv_heads"] * self.cfg["head_dim"]
        k = np.empty((count, kvd), np.uint16)
        v = np.empty((count, kvd), np.uint16)
        _check(lib().uq_model_kv(self.handle, layer, count, k.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                                 v.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))))
        return k, v

    def free(self):
        if getattr(self, "handle", None):
            lib().uq_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---------------------------------------------------------------- MoE expert FFN
MOE_CONFIG = dict(dim=2048, ff=768, experts=128, top_k=8, expert_kind=KIND_Q3_K, shared_kind=KIND_Q8_0)


def synth_moe(cfg, seed):
    """Seeded MoE layer: per expert gate/up (ff x dim) and down (dim x ff) in the
    expert kind; shared expert in the shared kind; shared gate vector 0.05 N(0,1)."""
    D, F, k, sk = cfg["dim"], cfg["ff"], cfg["expert_kind"], cfg["shared_kind"]
    ex = []
    for e in range(cfg["experts"]):
        ex.append(tuple(synth_quant(k, tensor_seed(seed, "blk.0.ffn_%s_exps.%d" % (p, e)), rows, n)
                        for p, rows, n in (("gate", F, D), ("up", F, D), ("down", D, F))))
    shared = tuple(synth_quant(sk, tensor_seed(seed, "blk.0.ffn_%s_shexp" % p), rows, n)
                   for p, rows, n in (("gate", F, D), ("up", F, D), ("down", D, F)))
    gate_inp = synth_normal(tensor_seed(seed, "blk.0.ffn_gate_inp_shexp"), D, 0.0, 0.05)
    return ex, shared, gate_inp


class MoeLayer:
    """Forward::ffn (frontier_forward.rs:164-199) over libuq (uq_moe_*)."""

    def __init__(self, cfg, experts, shared, gate_inp):
        self.cfg = dict(cfg)
        h = _vp()
        _check(lib().uq_moe_create(cfg["dim"], cfg["ff"], cfg["experts"], cfg["top_k"], cfg["expert_kind"],
                                   ctypes.byref(h)))
        self.handle = h
        for e, (g, u, d) in enumerate(experts):
            _check(lib().uq_moe_set_expert(h, e, g.ctypes.data, u.ctypes.data, d.ctypes.data))
        g, u, d = shared
        gi = None if gate_inp is None else np.ascontiguousarray(gate_inp, np.float32)
        _check(lib().uq_moe_set_shared(h, cfg["shared_kind"], g.ctypes.data, u.ctypes.data, d.ctypes.data,
                                       None if gi is None else _p(gi, _c_f32p)))

    @classmethod
    def from_gguf(cls, cfg, index, layer):
        """The layer's expert bank and shared expert read from a split model
        (uq_moe_load_gguf over a GgufIndex)."""
        self = cls.__new__(cls)
        self.cfg = dict(cfg)
        h = _vp()
        _check(lib().uq_moe_create(cfg["dim"], cfg["ff"], cfg["experts"], cfg["top_k"], cfg["expert_kind"],
                                   ctypes.byref(h)))
        self.handle = h
        _check(lib().uq_moe_load_gguf(h, index.handle, layer))
        return self

    def ffn(self, x, logits):
        x = np.ascontiguousarray(x, np.float32)
        lg = np.ascontiguousarray(logits, np.float32)
        out = np.empty(self.cfg["dim"], np.float32)
        ids = np.empty(self.cfg["top_k"], np.int32)
        w = np.empty(self.cfg["top_k"], np.float32)
        _check(lib().uq_moe_ffn(self.handle, _p(x, _c_f32p), _p(lg, _c_f32p), _p(out, _c_f32p), _p(ids, _c_i32p),
                                _p(w, _c_f32p)))
        return out, ids, w

    def ffn_dev(self, x_dev, logits_dev, out_dev, stream=None):
        _check(lib().uq_moe_ffn_dev(self.handle, x_dev, logits_dev, out_dev, stream))

    def run(self, xs, logits):
        """Timed back-to-back steps over host arrays xs [steps][dim], logits [steps][experts]."""
        xs = np.ascontiguousarray(xs, np.float32)
        logits = np.ascontiguousarray(logits, np.float32)
        steps = xs.shape[0]
        L = lib()
        bufs = []
        for a in (xs, logits, np.empty_like(xs)):
            p = _vp()
            _check(L.uq_dev_alloc(a.nbytes, ctypes.byref(p)))
            bufs.append(p)
        try:
            _check(L.uq_memcpy_h2d(bufs[0], xs.ctypes.data, xs.nbytes))
            _check(L.uq_memcpy_h2d(bufs[1], logits.ctypes.data, logits.nbytes))
            ms = ctypes.c_double()
            _check(L.uq_moe_run(self.handle, bufs[0], bufs[1], bufs[2], steps, ctypes.byref(ms)))
            out = np.empty_like(xs)
            _check(L.uq_memcpy_d2h(out.ctypes.data, bufs[2], out.nbytes))
        finally:
            for p in bufs:
                L.uq_dev_free(p)
        return out, ms.value

    def free(self):
        if getattr(self, "handle", None):
            lib().uq_moe_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def device_memory():
    f, t = ctypes.c_size_t(), ctypes.c_size_t()
    _check(lib().uq_device_memory(ctypes.byref(f), ctypes.byref(t)))
    return f.value, t.value


# ---------------------------------------------------------------- GGUF files
class GgufError(UqError):
    """A malformed GGUF directory; .gguf_error is the reference's error category
    (frontier_gguf.rs:7-8): one of GGUF_ERRORS."""

    def __init__(self, status, msg, gguf_error):
        super().__init__(status, msg)
        self.gguf_error = GGUF_ERRORS.get(gguf_error, gguf_error)


GGUF_ERRORS = {1: "Truncated", 2: "Magic", 3: "Version", 4: "Limit", 5: "Type", 6: "Utf8", 7: "Alignment",
               8: "Shape", 9: "Overflow", 10: "TensorBounds", 11: "Overlap", 12: "Duplicate", 13: "Missing",
               14: "Split"}


class Gguf:
    """A parsed GGUF directory (Shard, frontier_gguf.rs:104-200): from bytes
    with parse(), or from a file with open()."""

    def __init__(self, handle):
        self.handle = handle

    @classmethod
    def parse(cls, prefix, logical_bytes):
        buf = bytes(prefix)
        h, ge = _vp(), ctypes.c_int(0)
        rc = lib().uq_gguf_parse(buf, len(buf), logical_bytes, ctypes.byref(h), ctypes.byref(ge))
        if rc != OK:
            raise GgufError(rc, lib().uq_last_error().decode(errors="replace"), ge.value)
        return cls(h)

    @classmethod
    def open(cls, path):
        h, ge = _vp(), ctypes.c_int(0)
        rc = lib().uq_gguf_open(os.fsencode(path), ctypes.byref(h), ctypes.byref(ge))
        if rc != OK:
            raise GgufError(rc, lib().uq_last_error().decode(errors="replace"), ge.value)
        return cls(h)

    def free(self):
        if self.handle:
            lib().uq_gguf_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @property
    def data_offset(self):
        return lib().uq_gguf_data_offset(self.handle)

    def split(self):
        a, b, c = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        _check(lib().uq_gguf_split_info(self.handle, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)))
        return a.value, b.value, c.value

    def tensors(self):
        out = []
        for i in range(lib().uq_gguf_tensor_count(self.handle)):
            name, kind, rank = ctypes.c_char_p(), ctypes.c_uint32(), ctypes.c_int32()
            dims, off, nb = (ctypes.c_uint64 * 4)(), ctypes.c_uint64(), ctypes.c_uint64()
            _check(lib().uq_gguf_tensor_info(self.handle, i, ctypes.byref(name), ctypes.byref(kind), ctypes.byref(rank),
                                             dims, ctypes.byref(off), ctypes.byref(nb)))
            out.append({"name": name.value.decode(), "kind": kind.value, "dims": list(dims)[:rank.value],
                        "offset": off.value, "bytes": nb.value})
        return out

    def _ranged(self, fn, *args):
        off, n, ge = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_int(0)
        rc = fn(self.handle, *args, ctypes.byref(off), ctypes.byref(n), ctypes.byref(ge))
        if rc != OK:
            raise GgufError(rc, lib().uq_last_error().decode(errors="replace"), ge.value)
        return off.value, n.value

    def rows(self, index, start, count):
        """Tensor::rows: (absolute offset, bytes) of `count` rows from `start`."""
        return self._ranged(lib().uq_gguf_tensor_rows, index, start, count)

    def expert(self, index, expert):
        """Tensor::expert: (absolute offset, bytes) of one expert of a rank-3 tensor."""
        return self._ranged(lib().uq_gguf_tensor_expert, index, expert)

    def load_weight(self, index, expert=-1):
        """The tensor (or one expert's rows) as a device Weight."""
        t = self.tensors()[index]
        h = _vp()
        _check(lib().uq_gguf_load_weight(self.handle, index, expert, ctypes.byref(h)))
        w = Weight.__new__(Weight)
        w.kind, w.n = t["kind"], t["dims"][0]
        w.m = (t["dims"][1] if expert >= 0 else int(np.prod(t["dims"][1:]))) if len(t["dims"]) > 1 else 1
        w.handle = h
        return w

    def find(self, name):
        return lib().uq_gguf_find_tensor(self.handle, name.encode())

    def u64(self, key):
        v = ctypes.c_uint64()
        _check(lib().uq_gguf_meta_u64(self.handle, key.encode(), ctypes.byref(v)))
        return v.value

    def f32(self, key):
        v = ctypes.c_float()
        _check(lib().uq_gguf_meta_f32(self.handle, key.encode(), ctypes.byref(v)))
        return v.value

    def string(self, key):
        p, n = _vp(), ctypes.c_uint64()
        _check(lib().uq_gguf_meta_str(self.handle, key.encode(), ctypes.byref(p), ctypes.byref(n)))
        return ctypes.string_at(p.value, n.value).decode()

    def array(self, key):
        k, n = ctypes.c_uint32(), ctypes.c_uint64()
        _check(lib().uq_gguf_meta_array(self.handle, key.encode(), ctypes.byref(k), ctypes.byref(n)))
        return k.value, n.value

    def array_string(self, key, index):
        """Element `index` of a string-array value, as bytes."""
        p, n = _vp(), ctypes.c_uint64()
        _check(lib().uq_gguf_meta_array_str(self.handle, key.encode(), index, ctypes.byref(p), ctypes.byref(n)))
        return ctypes.string_at(p.value, n.value)

    def token_bytes(self, token_id):
        """Model::text (llm.rs:87-99) before the UTF-8 step: the token's bytes."""
        n = ctypes.c_uint64()
        buf = ctypes.create_string_buffer(256)
        rc = lib().uq_gguf_token_text(self.handle, token_id, buf, 256, ctypes.byref(n))
        if rc != 0 and n.value > 256:
            buf = ctypes.create_string_buffer(n.value)
            rc = lib().uq_gguf_token_text(self.handle, token_id, buf, n.value, ctypes.byref(n))
        _check(rc)
        return buf.raw[:n.value]

    def text(self, token_id):
        """Model::text: the token's bytes as text, invalid UTF-8 replaced (from_utf8_lossy)."""
        return self.token_bytes(token_id).decode("utf-8", errors="replace")

    def qwen2_config(self, max_seq=0):
        c = Qwen2Config()
        _check(lib().uq_gguf_qwen2_config(self.handle, max_seq, ctypes.byref(c)))
        return c.as_dict()


class GgufIndex:
    """ModelIndex (frontier_gguf.rs:101-137) over the Gguf shards of one split
    model; the shards must outlive the index."""

    def __init__(self, shards):
        self.shards_in = list(shards)
        arr = (_vp * len(self.shards_in))(*[g.handle for g in self.shards_in])
        h, ge = _vp(), ctypes.c_int(0)
        rc = lib().uq_gguf_index_create(arr, len(self.shards_in), ctypes.byref(h), ctypes.byref(ge))
        if rc != OK:
            raise GgufError(rc, lib().uq_last_error().decode(errors="replace"), ge.value)
        self.handle = h
        by_handle = {g.handle.value if hasattr(g.handle, "value") else g.handle: g for g in self.shards_in}
        self.shards = [by_handle[lib().uq_gguf_index_shard(h, i)] for i in range(lib().uq_gguf_index_shard_count(h))]

    def find(self, name):
        """ModelIndex::tensor: (shard position in split order, tensor index)."""
        sh, ix, ge = ctypes.c_int(), _i64(), ctypes.c_int(0)
        rc = lib().uq_gguf_index_find(self.handle, name.encode(), ctypes.byref(sh), ctypes.byref(ix), ctypes.byref(ge))
        if rc != OK:
            raise GgufError(rc, lib().uq_last_error().decode(errors="replace"), ge.value)
        return sh.value, ix.value

    def inventory(self):
        out, ge = (ctypes.c_uint64 * 3)(), ctypes.c_int(0)
        rc = lib().uq_gguf_index_inventory(self.handle, out, ctypes.byref(ge))
        if rc != OK:
            raise GgufError(rc, lib().uq_last_error().decode(errors="replace"), ge.value)
        return list(out)

    def free(self):
        if getattr(self, "handle", None):
            lib().uq_gguf_index_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
