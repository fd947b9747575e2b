"""uq_matvec_static (the entry point that allocates nothing: its quantized
activation lives in a static device scratch) against uq_matvec, through the C
ABI: bit-identical outputs on two calls in a row, the second with a smaller
input, so the scratch still holds the first call's longer activation."""
import ctypes

import numpy as np
import pytest

import uq

pytestmark = pytest.mark.gpu


def _dev(nbytes):
    p = ctypes.c_void_p()
    uq._check(uq.lib().uq_dev_alloc(nbytes, ctypes.byref(p)))
    return p


def _static(w, x):
    L = uq.lib()
    dx, dy = _dev(4 * x.size), _dev(4 * w.m)
    try:
        uq._check(L.uq_memcpy_h2d(dx, x.ctypes.data, 4 * x.size))
        uq._check(L.uq_matvec_static(w.handle, dx, dy, None))
        y = np.empty(w.m, np.float32)
        uq._check(L.uq_memcpy_d2h(y.ctypes.data, dy, 4 * w.m))   # synchronous on the library stream
    finally:
        L.uq_dev_free(dx)
        L.uq_dev_free(dy)
    return y


@pytest.mark.parametrize("kind,calls", [
    (uq.KIND_Q8_0, [(300, 16384), (1536, 1536)]),      # the scratch's maximum n, then a shorter x
    (uq.KIND_Q4_K, [(8960, 1536), (37, 512)]),
    (uq.KIND_Q3_K, [(768, 2048), (45, 768)]),
])
def test_matvec_static_equals_matvec(gpu, kind, calls):
    for i, (m, n) in enumerate(calls):
        w = uq.Weight(kind, n, m, uq.synth_quant(kind, 0x5A7 + 17 * i + kind, m, n))
        x = uq.synth_normal(0x5A8 + i + kind, n, 0.0, 2.0)
        try:
            y = _static(w, x)
            ref = uq.matvec(w, x)
            assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), (kind, m, n)
        finally:
            w.free()


def test_matvec_static_rejects_bad_calls(gpu):
    L = uq.lib()
    w = uq.Weight(uq.KIND_Q8_0, 64, 2, uq.synth_quant(uq.KIND_Q8_0, 3, 2, 64))
    try:
        assert L.uq_matvec_static(None, None, None, None) == uq.Error.ARG
        assert L.uq_matvec_static(w.handle, None, None, None) == uq.Error.ARG
    finally:
        w.free()
    f = uq.Weight(uq.KIND_F32, 64, 2, np.zeros(128, np.float32).view(np.uint8))
    dx, dy = _dev(256), _dev(8)
    try:
        assert L.uq_matvec_static(f.handle, dx, dy, None) == uq.Error.QUANT_TYPE
    finally:
        f.free()
        L.uq_dev_free(dx)
        L.uq_dev_free(dy)
