"""The C-ABI boundary on the CPU: libuq.so loads, exports every function the
headers declare, rejects calls before uq_init, and the host-only pieces
(row sizes, synthetic generators) behave. No GPU compute is issued here."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

import uq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(uq_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_library_exports_every_declared_function():
    L = uq.lib()
    names = header_functions()
    assert len(names) > 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the Python binding declares a signature for each exported function
    assert set(names) <= set(uq.declared_symbols()) | {"uq_stream"}


def test_calls_before_init_fail_cleanly():
    L = uq.lib()
    x = np.zeros(32, np.float32)
    y = np.zeros(4, np.float32)
    rc = L.uq_matvec(None, x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), 32,
                     y.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), 4)
    assert rc == uq.Error.ARG
    assert b"uq_init" in L.uq_last_error()
    assert L.uq_sync() == uq.Error.ARG


def test_row_bytes():
    assert uq.row_bytes(uq.KIND_Q8_0, 1536) == 1632
    assert uq.row_bytes(uq.KIND_Q4_K, 8960) == 35 * 144
    assert uq.row_bytes(uq.KIND_Q3_K, 2048) == 8 * 110
    assert uq.row_bytes(uq.KIND_F32, 7) == 28
    assert uq.row_bytes(uq.KIND_Q4_K, 640) == uq.Error.SHAPE
    assert uq.row_bytes(99, 256) == uq.Error.QUANT_TYPE


@pytest.mark.parametrize("kind,n", [(uq.KIND_Q8_0, 1536), (uq.KIND_Q4_K, 1536), (uq.KIND_Q3_K, 2048)])
def test_synth_is_deterministic_and_row_parallel(kind, n):
    a = uq.synth_quant(kind, 77, 300, n)
    b = uq.synth_quant(kind, 77, 300, n)
    assert np.array_equal(a, b)
    # row r does not depend on how many rows were requested (per-row streams)
    c = uq.synth_quant(kind, 77, 5, n)
    assert np.array_equal(a[:c.size], c)
    assert not np.array_equal(a, uq.synth_quant(kind, 78, 300, n))


def test_synth_distributions():
    import ggml_layouts as G
    rows, n = 512, 1536
    raw = uq.synth_quant(uq.KIND_Q8_0, 5, rows, n)
    d, q = G.q8_0_fields(raw, rows, n)
    assert q.min() == -127 and q.max() == 127
    assert abs(q.astype(np.float64).mean()) < 0.3
    ds = G.f16_to_f32(d).astype(np.float64)
    assert abs(np.median(ds) - 0.01) < 0.0005
    assert abs(np.log(ds).std() - 0.5) < 0.02
    x = uq.synth_normal(9, 200000)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    t = uq.synth_tokens(3, 100000, 151936)
    assert t.max() < 151936 and t.min() >= 0 and len(np.unique(t)) > 40000
    raw = uq.synth_quant(uq.KIND_Q4_K, 5, 8, 1536).reshape(-1, 144)
    un = [G.q4_k_unpack(b) for b in raw]
    assert max(u[4].max() for u in un) == 15 and min(u[4].min() for u in un) == 0
    assert max(u[2].max() for u in un) <= 63 and max(u[3].max() for u in un) <= 63
    raw = uq.synth_quant(uq.KIND_Q3_K, 5, 8, 2048).reshape(-1, 110)
    un = [G.q3_k_unpack(b) for b in raw]
    assert max(u[0].max() for u in un) == 3 and min(u[0].min() for u in un) == -4
    assert max(u[1].max() for u in un) == 63 and min(u[1].min() for u in un) == 0
