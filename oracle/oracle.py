"""ctypes binding of the CPU oracle (oracle/liboracle.so) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product (uefi-gpu_amd/) never does.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, Q8_0, Q3_K, Q4_K = 0, 8, 11, 12
Q6_K, IQ3_XXS, IQ4_NL, IQ4_XS, BF16 = 14, 18, 20, 23, 30
FRONTIER_KINDS = (F32, BF16, Q8_0, Q6_K, IQ3_XXS, IQ4_NL, IQ4_XS)

_lib = None
_f32p = ctypes.POINTER(ctypes.c_float)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i64 = ctypes.c_int64


class Layer(ctypes.Structure):
    _fields_ = [(n, _f32p) for n in ("attn_norm", "ffn_norm", "bq", "bk", "bv")] + \
               [(n, _u8p) for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")]


class Qwen2(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("layers", "dim", "hidden", "heads", "kv_heads", "head_dim",
                                             "vocab", "max_seq")] + \
               [("eps", ctypes.c_float), ("theta", ctypes.c_float),
                ("tok_embd", _u8p), ("output_norm", _f32p), ("output", _u8p), ("layer", ctypes.POINTER(Layer))]


class Moe(ctypes.Structure):
    _fields_ = [("dim", ctypes.c_int32), ("ff", ctypes.c_int32), ("experts", ctypes.c_int32),
                ("top_k", ctypes.c_int32), ("expert_kind", ctypes.c_uint32),
                ("gate", ctypes.POINTER(_u8p)), ("up", ctypes.POINTER(_u8p)), ("down", ctypes.POINTER(_u8p)),
                ("shared_kind", ctypes.c_uint32), ("sh_gate", _u8p), ("sh_up", _u8p), ("sh_down", _u8p),
                ("sh_scale", _f32p)]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def use_cpu_baseline_build():
    """Load liboracle_cpu.so (-O2, no OpenMP: one thread) instead of the tests'
    build. bench.py's CPU baseline calls this before any other oracle call."""
    global LIB_PATH
    if _lib is not None and LIB_PATH != os.path.join(HERE, "liboracle_cpu.so"):
        raise RuntimeError("oracle library already loaded")
    LIB_PATH = os.path.join(HERE, "liboracle_cpu.so")


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "uqo_set_threads": (None, [ctypes.c_int]),
            "uqo_get_threads": (ctypes.c_int, []),
            "uqo_half": (ctypes.c_float, [ctypes.c_uint16]),
            "uqo_f16_rne": (ctypes.c_uint16, [ctypes.c_float]),
            "uqo_expf": (ctypes.c_float, [ctypes.c_float]),
            "uqo_row_bytes": (_i64, [ctypes.c_uint32, _i64]),
            "uqo_dequantize": (ctypes.c_int, [ctypes.c_uint32, _u8p, _i64, _f32p]),
            "uqo_iq3_grid": (ctypes.c_uint32, [ctypes.c_int]),
            "uqo_iq4_value": (ctypes.c_int, [ctypes.c_int]),
            "uqo_linear": (None, [ctypes.c_uint32, _u8p, _i64, _i64, _f32p, _f32p]),
            "uqo_linear_f32seq": (None, [ctypes.c_uint32, _u8p, _i64, _i64, _f32p, _f32p]),
            "uqo_frontier_fixture": (_i64, [ctypes.c_uint32, _i64, _u8p]),
            "uqo_quant_act": (None, [_f32p, _i64, _f32p, _i8p]),
            "uqo_q8_block_dots": (None, [_u8p, _i64, _i64, _i8p, _i32p]),
            "uqo_q4k_block_dots": (None, [_u8p, _i64, _i64, _i8p, _i32p]),
            "uqo_q3k_block_dots": (None, [_u8p, _i64, _i64, _i8p, _i32p]),
            "uqo_matvec": (None, [ctypes.c_uint32, _u8p, _i64, _i64, _f32p, _i8p, _f32p]),
            "uqo_matvec_x": (None, [ctypes.c_uint32, _u8p, _i64, _i64, _f32p, _f32p]),
            "uqo_q8_matvec_f32seq": (None, [_u8p, _i64, _i64, _f32p, _f32p]),
            "uqo_q8_dequant_dot": (None, [_u8p, _i64, _i64, _f32p, _f32p]),
            "uqo_prefill_gemm": (None, [_u8p, _i64, _i64, _i64, _f32p, _i8p, _f32p]),
            "uqo_rmsnorm": (None, [_f32p, _f32p, _i64, ctypes.c_float, _f32p]),
            "uqo_rope_table": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_float, _f32p]),
            "uqo_rope_bias": (None, [_f32p, _f32p, ctypes.c_int, ctypes.c_int, _f32p]),
            "uqo_silu_mul": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
            "uqo_attention": (None, [_f32p, _u16p, _u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]),
            "uqo_greedy": (ctypes.c_int, [_f32p, _i64, ctypes.POINTER(ctypes.c_int)]),
            "uqo_state_new": (ctypes.c_void_p, [ctypes.POINTER(Qwen2)]),
            "uqo_state_free": (None, [ctypes.c_void_p]),
            "uqo_prefill": (ctypes.c_int, [ctypes.c_void_p, _u32p, ctypes.c_int, _u32p, _f32p]),
            "uqo_decode": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, _u32p, _f32p]),
            "uqo_state_keys": (_u16p, [ctypes.c_void_p, ctypes.c_int]),
            "uqo_state_values": (_u16p, [ctypes.c_void_p, ctypes.c_int]),
            "uqo_refo_new": (ctypes.c_void_p, [ctypes.POINTER(Qwen2), ctypes.c_int]),
            "uqo_refo_free": (None, [ctypes.c_void_p]),
            "uqo_refo_decode": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, _u32p, _f32p]),
            "uqo_refo_resnorm": (None, [_f32p, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_float, ctypes.c_int]),
            "uqo_refo_dotrow": (ctypes.c_float, [_u8p, _f32p, _i8p, _i64]),
            "uqo_refo_linear_row": (ctypes.c_float, [_u8p, _f32p, _i8p, _i64]),
            "uqo_refo_attention_head": (None, [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, _f32p]),
            "uqo_moe_route": (ctypes.c_int, [_f32p, ctypes.c_int, ctypes.c_int, _i32p, _f32p]),
            "uqo_moe_ffn": (ctypes.c_int, [ctypes.POINTER(Moe), _f32p, _f32p, _f32p, _i32p, _f32p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def p(a, ct):
    return a.ctypes.data_as(ct)


def set_threads(n):
    lib().uqo_set_threads(n)


def half(h):
    return lib().uqo_half(h)


def f16_rne(f):
    return lib().uqo_f16_rne(f)


def expf(x):
    return lib().uqo_expf(x)


def quant_act(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    s = np.empty(x.size // 32, np.float32)
    q = np.empty(x.size, np.int8)
    lib().uqo_quant_act(p(x, _f32p), x.size, p(s, _f32p), p(q, _i8p))
    return q, s


def block_dots(kind, w, n, m, qx):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    qx = np.ascontiguousarray(qx, dtype=np.int8)
    bsz = 16 if kind == Q3_K else 32
    d = np.empty(m * (n // bsz), np.int32)
    fn = {Q8_0: lib().uqo_q8_block_dots, Q4_K: lib().uqo_q4k_block_dots, Q3_K: lib().uqo_q3k_block_dots}[kind]
    fn(p(w, _u8p), n, m, p(qx, _i8p), p(d, _i32p))
    return d.reshape(m, n // bsz)


def matvec(kind, w, n, m, x):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(m, np.float32)
    lib().uqo_matvec_x(kind, p(w, _u8p), n, m, p(x, _f32p), p(y, _f32p))
    return y


def matvec_q(kind, w, n, m, xs, qx):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    y = np.empty(m, np.float32)
    lib().uqo_matvec(kind, p(w, _u8p), n, m, p(np.ascontiguousarray(xs, np.float32), _f32p),
                     p(np.ascontiguousarray(qx, np.int8), _i8p), p(y, _f32p))
    return y


def q8_matvec_f32seq(w, n, m, x):
    y = np.empty(m, np.float32)
    lib().uqo_q8_matvec_f32seq(p(np.ascontiguousarray(w, np.uint8), _u8p), n, m,
                               p(np.ascontiguousarray(x, np.float32), _f32p), p(y, _f32p))
    return y


def q8_dequant_dot(w, n, m, x):
    y = np.empty(m, np.float32)
    lib().uqo_q8_dequant_dot(p(np.ascontiguousarray(w, np.uint8), _u8p), n, m,
                             p(np.ascontiguousarray(x, np.float32), _f32p), p(y, _f32p))
    return y


def dequantize(kind, w, n):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.empty(n, np.float32)
    rc = lib().uqo_dequantize(kind, p(w, _u8p), n, p(out, _f32p))
    if rc:
        raise ValueError("dequantize rc=%d" % rc)
    return out


def row_bytes(kind, n):
    return lib().uqo_row_bytes(kind, n)


def iq3_grid():
    return np.array([lib().uqo_iq3_grid(i) for i in range(256)], np.uint32)


def iq4_values():
    return np.array([lib().uqo_iq4_value(i) for i in range(16)], np.int32)


def linear(kind, w, n, m, x):
    """fp32-activation matvec (frontier_matvec), exact double sum per row."""
    y = np.empty(m, np.float32)
    lib().uqo_linear(kind, p(np.ascontiguousarray(w, np.uint8), _u8p), n, m,
                     p(np.ascontiguousarray(x, np.float32), _f32p), p(y, _f32p))
    return y


def linear_f32seq(kind, w, n, m, x):
    """The reference's literal f32 sequential CPU check of frontier_matvec."""
    y = np.empty(m, np.float32)
    lib().uqo_linear_f32seq(kind, p(np.ascontiguousarray(w, np.uint8), _u8p), n, m,
                            p(np.ascontiguousarray(x, np.float32), _f32p), p(y, _f32p))
    return y


def frontier_fixture(kind, n):
    """The reference's synthetic quant bytes for `n` values (frontier_gpu.rs:37-50)."""
    rb = row_bytes(kind, n)
    if rb < 0:
        raise ValueError("bad kind/n")
    out = np.empty(rb, np.uint8)
    lib().uqo_frontier_fixture(kind, n, p(out, _u8p))
    return out


def prefill_gemm(w, n, m, xs, qx, batch):
    y = np.empty(batch * m, np.float32)
    lib().uqo_prefill_gemm(p(np.ascontiguousarray(w, np.uint8), _u8p), n, m, batch,
                           p(np.ascontiguousarray(xs, np.float32), _f32p),
                           p(np.ascontiguousarray(qx, np.int8), _i8p), p(y, _f32p))
    return y.reshape(batch, m)


def rmsnorm(x, gamma, eps=1e-6):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().uqo_rmsnorm(p(x, _f32p), p(np.ascontiguousarray(gamma, np.float32), _f32p), x.size, eps, p(y, _f32p))
    return y


def rope_table(seq, head_dim, theta):
    t = np.empty(seq * head_dim, np.float32)
    lib().uqo_rope_table(seq, head_dim, theta, p(t, _f32p))
    return t.reshape(seq, head_dim)


def rope_bias(v, bias, heads, head_dim, trig_row):
    v = np.array(v, dtype=np.float32, copy=True)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().uqo_rope_bias(p(v, _f32p), None if b is None else p(b, _f32p), heads, head_dim,
                        p(np.ascontiguousarray(trig_row, np.float32), _f32p))
    return v


def silu_mul(g, u):
    return lib().uqo_silu_mul(g, u)


def attention(q, keys, values, pos, heads, kv_heads, head_dim):
    out = np.empty(heads * head_dim, np.float32)
    lib().uqo_attention(p(np.ascontiguousarray(q, np.float32), _f32p),
                        p(np.ascontiguousarray(keys, np.uint16), _u16p),
                        p(np.ascontiguousarray(values, np.uint16), _u16p), pos, heads, kv_heads, head_dim,
                        p(out, _f32p))
    return out


def greedy(logits):
    bad = ctypes.c_int()
    i = lib().uqo_greedy(p(np.ascontiguousarray(logits, np.float32), _f32p), len(logits), ctypes.byref(bad))
    return i, bool(bad.value)


def moe_route(logits, top_k):
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(top_k, np.int32)
    w = np.empty(top_k, np.float32)
    rc = lib().uqo_moe_route(p(logits, _f32p), logits.size, top_k, p(ids, _i32p), p(w, _f32p))
    return rc, ids, w


class Model:
    """Oracle Qwen2 decoder over GGUF-layout numpy tensors (dict name -> array)."""

    def __init__(self, cfg, tensors):
        self.cfg = cfg
        self.t = tensors  # keep arrays alive
        L = cfg["layers"]
        self.layers = (Layer * L)()
        for i in range(L):
            g = lambda s: tensors["blk.%d.%s" % (i, s)]
            ly = self.layers[i]
            for f, nm in (("attn_norm", "attn_norm.weight"), ("ffn_norm", "ffn_norm.weight")):
                setattr(ly, f, p(g(nm), _f32p))
            for f, nm in (("bq", "attn_q.bias"), ("bk", "attn_k.bias"), ("bv", "attn_v.bias")):
                b = tensors.get("blk.%d.%s" % (i, nm))  # a model may carry no bias (NULL)
                setattr(ly, f, None if b is None else p(b, _f32p))
            for f, nm in (("wq", "attn_q.weight"), ("wk", "attn_k.weight"), ("wv", "attn_v.weight"),
                          ("wo", "attn_output.weight"), ("wg", "ffn_gate.weight"), ("wu", "ffn_up.weight"),
                          ("wd", "ffn_down.weight")):
                setattr(ly, f, p(g(nm), _u8p))
        self.m = Qwen2(layers=L, dim=cfg["dim"], hidden=cfg["hidden"], heads=cfg["heads"],
                       kv_heads=cfg["kv_heads"], head_dim=cfg["head_dim"], vocab=cfg["vocab"],
                       max_seq=cfg["max_seq"], eps=cfg["eps"], theta=cfg["theta"],
                       tok_embd=p(tensors["token_embd.weight"], _u8p),
                       output_norm=p(tensors["output_norm.weight"], _f32p),
                       output=p(tensors["output.weight"], _u8p),
                       layer=ctypes.cast(self.layers, ctypes.POINTER(Layer)))
        self.state = lib().uqo_state_new(ctypes.byref(self.m))

    def __del__(self):
        if getattr(self, "state", None):
            lib().uqo_state_free(self.state)
            self.state = None

    def prefill(self, tokens, want_logits=False):
        tokens = np.ascontiguousarray(tokens, np.uint32)
        nxt = ctypes.c_uint32()
        logits = np.empty(self.cfg["vocab"], np.float32) if want_logits else None
        rc = lib().uqo_prefill(self.state, p(tokens, _u32p), tokens.size, ctypes.byref(nxt),
                               None if logits is None else p(logits, _f32p))
        return rc, nxt.value, logits

    def decode(self, token, pos, want_logits=False):
        nxt = ctypes.c_uint32()
        logits = np.empty(self.cfg["vocab"], np.float32) if want_logits else None
        rc = lib().uqo_decode(self.state, token, pos, ctypes.byref(nxt), None if logits is None else p(logits, _f32p))
        return rc, nxt.value, logits

    def keys(self, layer, count):
        kvd = self.cfg["kv_heads"] * self.cfg["head_dim"]
        ptr = lib().uqo_state_keys(self.state, layer)
        return np.ctypeslib.as_array(ptr, shape=(count * kvd,)).reshape(count, kvd).copy()

    def set_kv(self, layer, keys, values):
        """Overwrite positions [0, len(keys)) of one layer's caches (fp16 bits,
        [count][kv_heads*head_dim]), e.g. with a prefill computed elsewhere."""
        kvd = self.cfg["kv_heads"] * self.cfg["head_dim"]
        keys = np.ascontiguousarray(keys, np.uint16).reshape(-1, kvd)
        values = np.ascontiguousarray(values, np.uint16).reshape(-1, kvd)
        n = keys.shape[0]
        assert values.shape[0] == n <= self.cfg["max_seq"]
        for ptr, src in ((lib().uqo_state_keys(self.state, layer), keys),
                         (lib().uqo_state_values(self.state, layer), values)):
            np.ctypeslib.as_array(ptr, shape=(n * kvd,))[:] = src.reshape(-1)

    def values(self, layer, count):
        kvd = self.cfg["kv_heads"] * self.cfg["head_dim"]
        ptr = lib().uqo_state_values(self.state, layer)
        return np.ctypeslib.as_array(ptr, shape=(count * kvd,)).reshape(count, kvd).copy()


class RefoModel(Model):
    """The reference-order decoder: the f32 operation orders of the reference's
    decode-graph kernels (gpu_graph.rs:137-162), f32 KV cache (kv_fp16: the
    cache rounded to fp16 as the library stores it). Token by token only."""

    def __init__(self, cfg, tensors, kv_fp16=False):
        super().__init__(cfg, tensors)
        self.refo = lib().uqo_refo_new(ctypes.byref(self.m), 1 if kv_fp16 else 0)

    def __del__(self):
        if getattr(self, "refo", None):
            lib().uqo_refo_free(self.refo)
            self.refo = None
        super().__del__()

    def decode(self, token, pos, want_logits=False):
        nxt = ctypes.c_uint32()
        logits = np.empty(self.cfg["vocab"], np.float32) if want_logits else None
        rc = lib().uqo_refo_decode(self.refo, token, pos, ctypes.byref(nxt), None if logits is None else p(logits, _f32p))
        return rc, nxt.value, logits

    def prefill(self, tokens, want_logits=False):
        raise NotImplementedError("the reference-order decoder ingests prompts token by token")


def refo_resnorm(x, residual, w, eps=1e-6, add=True):
    """fused_resnorm (gpu_fused.cu:28-35): returns (x + residual, y)."""
    x = np.ascontiguousarray(x, np.float32).copy()
    r = np.ascontiguousarray(residual, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    lib().uqo_refo_resnorm(p(x, _f32p), p(r, _f32p), p(w, _f32p), p(y, _f32p), x.size, eps, 1 if add else 0)
    return x, y


def refo_dotrow(w_row, xs, qx):
    """dotrow (gpu_dp4a.cu:32-39) of one Q8_0 row with a quantized x."""
    return lib().uqo_refo_dotrow(p(np.ascontiguousarray(w_row, np.uint8), _u8p),
                                 p(np.ascontiguousarray(xs, np.float32), _f32p),
                                 p(np.ascontiguousarray(qx, np.int8), _i8p), qx.size // 32)


def refo_linear_row(w_row, xs, qx):
    """linear_dp4a (gpu_dp4a.cu:40-52) of one Q8_0 row with a quantized x."""
    return lib().uqo_refo_linear_row(p(np.ascontiguousarray(w_row, np.uint8), _u8p),
                                     p(np.ascontiguousarray(xs, np.float32), _f32p),
                                     p(np.ascontiguousarray(qx, np.int8), _i8p), qx.size // 32)


def refo_attention_head(q, keys, values, pos, kh, hd):
    """fused_attention (gpu_attention.cu:2-26) for one head over f32 [t][kvd] caches."""
    keys = np.ascontiguousarray(keys, np.float32)
    values = np.ascontiguousarray(values, np.float32)
    out = np.empty(hd, np.float32)
    lib().uqo_refo_attention_head(p(np.ascontiguousarray(q, np.float32), _f32p), p(keys, _f32p), p(values, _f32p),
                                  pos, keys.shape[1], kh, hd, p(out, _f32p))
    return out


class MoeLayer:
    """Oracle MoE FFN over GGUF-layout expert tensors."""

    def __init__(self, dim, ff, experts, top_k, expert_kind, gate, up, down, shared_kind, sh_gate, sh_up, sh_down,
                 sh_scale):
        self.keep = (gate, up, down, sh_gate, sh_up, sh_down, sh_scale)
        arr = lambda xs: (_u8p * len(xs))(*[p(x, _u8p) for x in xs])
        self.g, self.u, self.d = arr(gate), arr(up), arr(down)
        self.m = Moe(dim=dim, ff=ff, experts=experts, top_k=top_k, expert_kind=expert_kind,
                     gate=ctypes.cast(self.g, ctypes.POINTER(_u8p)), up=ctypes.cast(self.u, ctypes.POINTER(_u8p)),
                     down=ctypes.cast(self.d, ctypes.POINTER(_u8p)), shared_kind=shared_kind,
                     sh_gate=p(sh_gate, _u8p), sh_up=p(sh_up, _u8p), sh_down=p(sh_down, _u8p),
                     sh_scale=None if sh_scale is None else p(sh_scale, _f32p))

    def ffn(self, x, router_logits):
        out = np.empty(self.m.dim, np.float32)
        ids = np.empty(self.m.top_k, np.int32)
        w = np.empty(self.m.top_k, np.float32)
        rc = lib().uqo_moe_ffn(ctypes.byref(self.m), p(np.ascontiguousarray(x, np.float32), _f32p),
                               p(np.ascontiguousarray(router_logits, np.float32), _f32p), p(out, _f32p),
                               p(ids, _i32p), p(w, _f32p))
        return rc, out, ids, w
