"""GPU parity of the fp32-activation reader (frontier_dequant / frontier_matvec /
frontier_multi_matvec, driver/kernels/frontier_quant.cu:12-93) against the CPU
oracle, through the C ABI.

Dequant is bit-exact. Linear outputs are compared with the oracle's exactly
summed row (<= 1 ulp, and |gpu - oracle| <= 1e-3 * max(|oracle|, 1e-3 *
max|oracle|)) and with the reference's own check: an f32 sequential sum within
2e-4 + 2e-5 |ref| (frontier_gpu.rs:111). The job-table form must equal the
single-weight form bit for bit (frontier_gpu.rs:305, :401)."""
import numpy as np
import pytest

import oracle as O
import uq

pytestmark = pytest.mark.gpu

KINDS = list(uq.LINEAR_KINDS)


def tol_ok(y, ref):
    scale = np.abs(ref).max()
    return bool((np.abs(y - ref) <= 1e-3 * np.maximum(np.abs(ref), 1e-3 * scale)).all())


def ulps(a, b):
    a = a.view(np.int32).astype(np.int64)
    b = b.view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def ref_ok(y, seq):
    return bool((np.abs(y - seq) <= 2e-4 + 2e-5 * np.abs(seq)).all())


@pytest.mark.parametrize("kind", KINDS)
def test_dequant_reference_fixture_bit_exact(gpu, kind):
    # the reference's dequant probe: fixture(kind, 8192), frontier_gpu.rs:92-110
    n = 8192
    raw = O.frontier_fixture(kind, n)
    got = uq.dequantize(kind, raw, n)
    assert np.array_equal(got.view(np.uint32), O.dequantize(kind, raw, n).view(np.uint32))


@pytest.mark.parametrize("kind", KINDS)
def test_dequant_random_bit_exact(gpu, kind):
    n, rows = 2560, 37
    raw = uq.synth_quant(kind, 0xDE0 + kind, rows, n)
    got = uq.dequantize(kind, raw, n * rows)
    assert np.array_equal(got.view(np.uint32), O.dequantize(kind, raw, n * rows).view(np.uint32))


@pytest.mark.parametrize("kind", KINDS)
def test_linear_reference_probe(gpu, kind):
    # frontier_gpu.rs:92-110: n=2560, m=17, x = ((i % 29) - 14) / 32
    n, m = 2560, 17
    raw = O.frontier_fixture(kind, n * m)
    x = ((np.arange(n) % 29 - 14) / 32).astype(np.float32)
    w = uq.Weight(kind, n, m, raw)
    y = uq.linear(w, x)
    ref = O.linear(kind, raw, n, m, x)
    assert tol_ok(y, ref) and ulps(y, ref).max() <= 1
    assert ref_ok(y, O.linear_f32seq(kind, raw, n, m, x))


@pytest.mark.parametrize("kind,n,m", [(k, 2560, 1000) for k in KINDS] +
                         [(uq.KIND_IQ3_XXS, 2560, 640), (uq.KIND_IQ4_NL, 640, 2560), (uq.KIND_Q6_K, 2560, 3001),
                          (uq.KIND_Q8_0, 16384, 64), (uq.KIND_F32, 16384, 33), (uq.KIND_BF16, 8, 5),
                          (uq.KIND_IQ4_XS, 256, 7), (uq.KIND_IQ3_XXS, 16384, 9)])
def test_linear_random_shapes(gpu, kind, n, m):
    raw = uq.synth_quant(kind, 0x11EA + n + m + kind, m, n)
    x = uq.synth_normal(0x5EED + n, n)
    w = uq.Weight(kind, n, m, raw)
    y = uq.linear(w, x)
    ref = O.linear(kind, raw, n, m, x)
    assert tol_ok(y, ref)
    d = ulps(y, ref)
    assert d.max() <= 1 and (d == 0).mean() > 0.999, (d.max(), (d == 0).mean())


def wide_range_x(n, seed):
    """x whose 32-blocks exercise the exact-integer staging: zeros, denormals,
    a 2^20 range (double path), 1e30 beside 1e-30 (double path), small values
    with zero low bits beside a large one (integer path), -0.0, ordinary."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, n).astype(np.float32)
    x[0:32] = 0
    x[32:64] = (rng.normal(0, 1, 32) * 1e-41).astype(np.float32)          # denormals
    x[64:96] = rng.normal(0, 1, 32).astype(np.float32) * np.float32(2.0) ** rng.integers(-20, 1, 32)
    x[96:128] = rng.normal(0, 1, 32).astype(np.float32)
    x[96], x[97] = 1e30, -1e-30
    x[128:160] = (rng.integers(-8, 8, 32) * 2.0 ** -20).astype(np.float32)
    x[128] = 3.0e3
    x[160:192] = -0.0
    return x


@pytest.mark.parametrize("kind", [k for k in KINDS if k not in (uq.KIND_F32, uq.KIND_BF16)])
def test_linear_wide_range_blocks(gpu, kind):
    n, m = 2560, 300
    raw = uq.synth_quant(kind, 0x71DE + kind, m, n)
    x = wide_range_x(n, kind)
    w = uq.Weight(kind, n, m, raw)
    y = uq.linear(w, x)
    ref = O.linear(kind, raw, n, m, x)
    assert np.isfinite(y).all()
    assert ulps(y, ref).max() <= 1
    assert tol_ok(y, ref)


def test_multi_format_job_table(gpu):
    # frontier_gpu.rs:281-307: all seven kinds in one dispatch, non-four-row tails
    n = 2560
    pairs, raws = [], []
    for i, (kind, m) in enumerate([(0, 1), (30, 3), (8, 17), (14, 5), (18, 640), (20, 4), (23, 127)]):
        row = O.frontier_fixture(kind, n)
        raw = np.tile(row, m)
        x = np.sin(np.arange(n, dtype=np.float32) * np.float32(0.031) + np.float32(i * 0.173)).astype(np.float32)
        pairs.append((uq.Weight(kind, n, m, raw), x))
        raws.append((kind, raw, m, x))
    multi = uq.linear_batch(pairs)
    for (w, x), y, (kind, raw, m, _) in zip(pairs, multi, raws):
        single = uq.linear(w, x)
        assert np.array_equal(y.view(np.uint32), single.view(np.uint32))
        ref = O.linear(kind, raw, n, m, x)
        assert tol_ok(y, ref) and ulps(y, ref).max() <= 1
        assert ref_ok(y, O.linear_f32seq(kind, raw, n, m, x))


def test_expert_batch_rounds(gpu):
    # frontier_gpu.rs:367-410: gate/up IQ3_XXS (640 x 2560) and down IQ4_NL
    # (2560 x 640) jobs, counts 2..32, batch == serial bit for bit
    parts = []
    for p in range(3):
        n, m, kind = (640, 2560, uq.KIND_IQ4_NL) if p == 2 else (2560, 640, uq.KIND_IQ3_XXS)
        raw = uq.synth_quant(kind, 0xE0 + p, m, n)
        parts.append((uq.Weight(kind, n, m, raw), raw, kind, n, m))
    for rnd, count in enumerate([2, 3, 4, 11, 23, 32]):
        jobs = []
        for i in range(count):
            w, raw, kind, n, m = parts[i % 3]
            x = np.sin(np.arange(n, dtype=np.float32) * np.float32(0.031) +
                       np.float32((i + rnd * 7) * 0.17)).astype(np.float32)
            jobs.append((w, x))
        batch = uq.linear_batch(jobs)
        for i, ((w, x), y) in enumerate(zip(jobs, batch)):
            assert np.array_equal(y.view(np.uint32), uq.linear(w, x).view(np.uint32))
            _, raw, kind, n, m = parts[i % 3]
            if rnd == 0:
                ref = O.linear(kind, raw, n, m, x)
                assert tol_ok(y, ref) and ulps(y, ref).max() <= 1


def test_linear_device_form_matches_host_form(gpu):
    import ctypes
    kind, n, m = uq.KIND_IQ4_XS, 2560, 300
    raw = uq.synth_quant(kind, 77, m, n)
    w = uq.Weight(kind, n, m, raw)
    x = uq.synth_normal(78, n)
    dx, dy = ctypes.c_void_p(), ctypes.c_void_p()
    L = uq.lib()
    assert L.uq_dev_alloc(4 * n, ctypes.byref(dx)) == 0 and L.uq_dev_alloc(4 * m, ctypes.byref(dy)) == 0
    try:
        assert L.uq_memcpy_h2d(dx, x.ctypes.data, 4 * n) == 0
        assert L.uq_linear_dev(w.handle, dx, dy, None) == 0
        assert L.uq_sync() == 0
        y = np.empty(m, np.float32)
        assert L.uq_memcpy_d2h(y.ctypes.data, dy, 4 * m) == 0
    finally:
        L.uq_dev_free(dx)
        L.uq_dev_free(dy)
    assert np.array_equal(y.view(np.uint32), uq.linear(w, x).view(np.uint32))


def test_linear_errors(gpu):
    n, m = 512, 4
    q3 = uq.Weight(uq.KIND_Q3_K, n, m, uq.synth_quant(uq.KIND_Q3_K, 1, m, n))
    x = np.ones(n, np.float32)
    with pytest.raises(uq.UqError) as e:
        uq.linear(q3, x)
    assert e.value.status == uq.Error.QUANT_TYPE
    w = uq.Weight(uq.KIND_IQ4_NL, n, m, uq.synth_quant(uq.KIND_IQ4_NL, 2, m, n))
    bad = x.copy()
    bad[7] = np.nan
    with pytest.raises(uq.UqError) as e:
        uq.linear(w, bad)
    assert e.value.status == uq.Error.NONFINITE
    with pytest.raises(uq.UqError) as e:
        uq.linear(w, x[:256])
    assert e.value.status == uq.Error.SHAPE
    # an infinite fp16 scale gives a non-finite output (frontier_backend.rs:222)
    raw = uq.synth_quant(uq.KIND_IQ4_NL, 3, m, n)
    raw[0], raw[1] = 0x00, 0x7C
    with pytest.raises(uq.UqError) as e:
        uq.linear(uq.Weight(uq.KIND_IQ4_NL, n, m, raw), x)
    assert e.value.status == uq.Error.NONFINITE
    with pytest.raises(uq.UqError) as e:
        uq.dequantize(uq.KIND_Q6_K, np.zeros(209, np.uint8), 256)
    assert e.value.status == uq.Error.SHAPE
    with pytest.raises(uq.UqError) as e:
        uq.dequantize(99, np.zeros(256, np.uint8), 256)
    assert e.value.status == uq.Error.QUANT_TYPE
    with pytest.raises(uq.UqError) as e:
        uq.Weight(uq.KIND_BF16, 12, 2, np.zeros(48, np.uint8))
    assert e.value.status == uq.Error.SHAPE
    with pytest.raises(uq.UqError) as e:
        uq.matvec(w, x)          # int8-activation linears take Q8_0 / Q4_K / Q3_K only
    assert e.value.status == uq.Error.QUANT_TYPE
