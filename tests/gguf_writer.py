"""GGUF v3 writer for the tests (test-side data only; the library parses).

Layout (GGUF v3): magic "GGUF", u32 version, u64 tensor count, u64 metadata
count, metadata (string key, u32 type, value), tensor infos (string name, u32
rank, u64 dims, u32 type, u64 offset relative to the data section), data
section at the aligned end of the directory.
"""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}
# ggml type -> (block values, bytes per block)
TYPE_BLOCK = {0: (1, 4), 1: (1, 2), 8: (32, 34), 11: (256, 110), 12: (256, 144), 14: (256, 210), 18: (256, 98),
              20: (32, 18), 23: (256, 136), 30: (1, 2)}


def gstr(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value(kind, v):
    if kind == STRING:
        return gstr(v)
    if kind == ARRAY:
        elem, items = v
        return struct.pack("<IQ", elem, len(items)) + b"".join(value(elem, x) for x in items)
    return struct.pack(_FMT[kind], v)


def tensor_bytes(kind, dims):
    block, nb = TYPE_BLOCK[kind]
    n = dims[0] // block * nb
    for d in dims[1:]:
        n *= d
    return n


def directory(meta, infos, version=3, n_tensors=None, n_kv=None):
    """meta: [(key, kind, value)]; infos: [(name, dims, kind, offset)] -> bytes."""
    out = b"GGUF" + struct.pack("<IQQ", version, len(infos) if n_tensors is None else n_tensors,
                                len(meta) if n_kv is None else n_kv)
    for k, kind, v in meta:
        out += gstr(k) + struct.pack("<I", kind) + value(kind, v)
    for name, dims, kind, off in infos:
        out += gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", kind, off)
    return out


def write(meta, tensors, alignment=32):
    """tensors: [(name, dims, kind, data bytes)] -> whole file bytes (tensors packed in order)."""
    infos, off = [], 0
    for name, dims, kind, data in tensors:
        assert len(data) == tensor_bytes(kind, dims)
        infos.append((name, dims, kind, off))
        off += (len(data) + alignment - 1) // alignment * alignment
    d = directory(meta, infos)
    d += b"\0" * (-len(d) % alignment)
    body = b""
    for name, dims, kind, data in tensors:
        body += data + b"\0" * (-len(data) % alignment)
    return d + body, len(d)


def synthetic(offsets, width):
    """The directory of frontier_gguf.rs:245-254: tensors "tensor.i", rank 2,
    dims [width, 2], Q8_0, at the given offsets; no metadata."""
    return directory([], [("tensor.%d" % i, [width, 2], 8, off) for i, off in enumerate(offsets)])


def qwen2_file(cfg, tensors, tie_output=False, extra_meta=()):
    """A Qwen2 GGUF from synth_qwen2-style tensors {name: (kind, n, rows, array)}."""
    meta = [("general.architecture", STRING, "qwen2"),
            ("qwen2.block_count", U32, cfg["layers"]),
            ("qwen2.context_length", U32, cfg["max_seq"]),
            ("qwen2.embedding_length", U32, cfg["dim"]),
            ("qwen2.feed_forward_length", U32, cfg["hidden"]),
            ("qwen2.attention.head_count", U32, cfg["heads"]),
            ("qwen2.attention.head_count_kv", U32, cfg["kv_heads"]),
            ("qwen2.rope.freq_base", F32, cfg["theta"]),
            ("qwen2.attention.layer_norm_rms_epsilon", F32, cfg["eps"]),
            ("tokenizer.ggml.tokens", ARRAY, (STRING, ["t%d" % i for i in range(16)]))] + list(extra_meta)
    ts = []
    for name, (kind, n, rows, arr) in tensors.items():
        if tie_output and name == "output.weight":
            continue
        dims = [n] if rows == 1 and kind == 0 else [n, rows]
        ts.append((name, dims, kind, arr.tobytes()))
    return write(meta, ts)
