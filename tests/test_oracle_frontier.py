"""Pins of the oracle's restatement of the reference's remaining quant kinds
(dequantize, driver/src/frontier_core.rs:53-106) and of its fp32-activation
linear (frontier_matvec, driver/kernels/frontier_quant.cu:58-66).

Each kind is checked against blocks built by an encoder written here from the
layout description (code, scale and sign placement), so a wrong shift, index
or multiply order in the oracle fails a known-answer case; plus the
reference's own row_bytes cases, the code book / grid invariants, fp16-scale
linearity and the reference's fixture generator restated in Python."""
import struct

import numpy as np
import pytest

import oracle as O

rng = np.random.default_rng(20260)


def f16(v):
    return np.float16(v).view(np.uint16).item()


# ---------------------------------------------------------------- encoders (layout -> bytes)
def enc_iq4_nl(d, codes):
    """One 18-byte block: fp16 d, then 16 bytes, code j in the low nibble of
    byte j (j < 16) or the high nibble of byte j-16."""
    b = bytearray(18)
    struct.pack_into("<H", b, 0, f16(d))
    for j, c in enumerate(codes):
        b[2 + j % 16] |= (c & 15) << (4 * (j // 16))
    return bytes(b)


def enc_iq4_xs(d, scales6, codes):
    """136-byte superblock: fp16 d, u16 scales_h (2 bits per sub-block), 4
    bytes scales_l (4 bits per sub-block), 8 x 16 bytes of nibbles."""
    b = bytearray(136)
    sh = 0
    for sb, s in enumerate(scales6):
        b[4 + sb // 2] |= (s & 15) << (4 * (sb % 2))
        sh |= ((s >> 4) & 3) << (2 * sb)
    struct.pack_into("<HH", b, 0, f16(d), sh)
    for j, c in enumerate(codes):
        sb, jj = j // 32, j % 32
        b[8 + sb * 16 + jj % 16] |= (c & 15) << (4 * (jj // 16))
    return bytes(b)


def enc_q6_k(d, scales, q):
    """210-byte superblock from codes q in [-32, 31] and 16 int8 scales:
    low 4 bits in ql, high 2 bits in qh, scales, fp16 d last."""
    b = bytearray(210)
    for j, v in enumerate(q):
        u = v + 32
        sub, g, l = j // 128, (j % 128) // 32, j % 32
        b[sub * 64 + l + (g % 2) * 32] |= (u & 15) << (4 * (g // 2))
        b[128 + sub * 32 + l] |= ((u >> 4) & 3) << (2 * g)
    for i, s in enumerate(scales):
        b[192 + i] = s & 255
    struct.pack_into("<H", b, 208, f16(d))
    return bytes(b)


def enc_iq3_xxs(d, idx, signs7, scale4):
    """98-byte superblock: fp16 d, 64 grid indices (one per 4 values), 8 words
    of 4 x 7 sign bits + a 4-bit scale in the top bits."""
    b = bytearray(98)
    struct.pack_into("<H", b, 0, f16(d))
    for i, v in enumerate(idx):
        b[2 + i] = v
    for sb in range(8):
        w = scale4[sb] << 28
        for g in range(4):
            w |= signs7[sb][g] << (7 * g)
        struct.pack_into("<I", b, 66 + 4 * sb, w)
    return bytes(b)


# ---------------------------------------------------------------- tables
def test_row_bytes_reference_cases():
    # frontier_core.rs:129-133
    assert O.row_bytes(O.IQ4_XS, 640) < 0
    assert O.row_bytes(O.IQ4_NL, 160) == 90
    assert O.row_bytes(O.IQ3_XXS, 2560) == 980
    assert O.row_bytes(99, 256) < 0
    assert O.row_bytes(O.Q6_K, 256) == 210 and O.row_bytes(O.BF16, 3) == 6 and O.row_bytes(O.F32, 3) == 12


def test_iq4_book_and_iq3_grid_invariants():
    book = O.iq4_values()
    assert book.size == 16 and (np.diff(book) > 0).all() and book[0] == -127 and book[-1] == 113
    grid = O.iq3_grid()
    levels = {4, 12, 20, 28, 36, 44, 52, 62}
    assert len(set(grid.tolist())) == 256 and (np.diff(grid.astype(np.int64)) > 0).all()
    assert all(((int(v) >> (8 * k)) & 255) in levels for v in grid for k in range(4))
    # first and last entries of the reference's table (frontier_tables.rs:3,34)
    assert grid[0] == 0x04040404 and grid[1] == 0x04040414 and grid[255] == 0x3E341C04


# ---------------------------------------------------------------- known answers
def test_bf16_and_f32():
    h = rng.integers(0, 65536, 4096).astype(np.uint16)
    h[(h & 0x7F80) == 0x7F80] = 0x3F80          # no inf/nan patterns
    out = O.dequantize(O.BF16, h.view(np.uint8), h.size)
    assert np.array_equal(out.view(np.uint32), h.astype(np.uint32) << 16)
    f = rng.normal(0, 1, 1000).astype(np.float32)
    assert np.array_equal(O.dequantize(O.F32, f.view(np.uint8), f.size), f)


@pytest.mark.parametrize("d", [1.0, 0.5, -0.0078125, 6.1035156e-05 * 0.25])
def test_iq4_nl_known_answer(d):
    book = O.iq4_values()
    codes = [int(c) for c in rng.integers(0, 16, 32)]
    out = O.dequantize(O.IQ4_NL, np.frombuffer(enc_iq4_nl(d, codes), np.uint8), 32)
    dd = np.float32(np.float16(d))
    assert np.array_equal(out, (dd * book[codes].astype(np.float32)).astype(np.float32))


def test_iq4_xs_known_answer():
    book = O.iq4_values()
    d = 0.03125
    scales = [0, 1, 31, 32, 33, 47, 62, 63]
    codes = [int(c) for c in rng.integers(0, 16, 256)]
    out = O.dequantize(O.IQ4_XS, np.frombuffer(enc_iq4_xs(d, scales, codes), np.uint8), 256)
    for j in range(256):
        # (d * (sc - 32)) * book[q], the f32 order of frontier_core.rs:85
        want = np.float32(np.float32(d) * np.float32(scales[j // 32] - 32)) * np.float32(book[codes[j]])
        assert out[j] == want, j


def test_q6_k_known_answer():
    d = 0.0009765625
    scales = [int(s) for s in rng.integers(-128, 128, 16)]
    q = [int(v) for v in rng.integers(-32, 32, 256)]
    q[:4] = [-32, 31, 0, -1]
    out = O.dequantize(O.Q6_K, np.frombuffer(enc_q6_k(d, scales, q), np.uint8), 256)
    want = (np.float32(d) * np.array(scales, np.float32)[np.arange(256) // 16]).astype(np.float32) * \
        np.array(q, np.float32)
    assert np.array_equal(out, want.astype(np.float32))


def test_iq3_xxs_known_answer_and_sign_parity():
    grid = O.iq3_grid()
    d = 0.25
    idx = [int(v) for v in rng.integers(0, 256, 64)]
    signs7 = [[int(v) for v in rng.integers(0, 128, 4)] for _ in range(8)]
    scale4 = [int(v) for v in rng.integers(0, 16, 8)]
    out = O.dequantize(O.IQ3_XXS, np.frombuffer(enc_iq3_xxs(d, idx, signs7, scale4), np.uint8), 256)
    for j in range(256):
        sb, g, t = j // 32, (j % 32) // 8, j % 8
        s7 = signs7[sb][g]
        s8 = s7 | ((bin(s7).count("1") & 1) << 7)     # 8th sign: even count of negatives
        mag = (int(grid[idx[j // 4]]) >> (8 * (j % 4))) & 255
        scale = np.float32(np.float32(np.float32(d) * np.float32(0.5 + scale4[sb])) * np.float32(0.5))
        want = np.float32(scale * np.float32(mag)) * np.float32(-1.0 if (s8 >> t) & 1 else 1.0)
        assert out[j] == want, j
    # every 8-group has an even number of negative values
    neg = (out < 0).reshape(32, 8).sum(axis=1)
    assert (neg % 2 == 0).all()


@pytest.mark.parametrize("kind", [O.Q8_0, O.Q6_K, O.IQ3_XXS, O.IQ4_NL, O.IQ4_XS])
def test_fp16_scale_linearity(kind):
    """Doubling every block's fp16 d (exponent + 1) doubles every value."""
    n = 512
    raw = O.frontier_fixture(kind, n)
    block, size, off = {O.Q8_0: (32, 34, 0), O.Q6_K: (256, 210, 208), O.IQ3_XXS: (256, 98, 0),
                        O.IQ4_NL: (32, 18, 0), O.IQ4_XS: (256, 136, 0)}[kind]
    dbl = raw.copy()
    for b in range(n // block):
        h = int(dbl[b * size + off]) | (int(dbl[b * size + off + 1]) << 8)
        h += 1 << 10
        dbl[b * size + off], dbl[b * size + off + 1] = h & 255, h >> 8
    a = O.dequantize(kind, raw, n)
    b2 = O.dequantize(kind, dbl, n)
    assert np.array_equal(b2, (a * np.float32(2)).astype(np.float32))


# ---------------------------------------------------------------- fixture + linear
def py_fixture(kind, n):
    """frontier_gpu.rs:37-50 restated independently of the C oracle."""
    rb = O.row_bytes(kind, n)
    out = bytearray(rb)
    st = 0x13243546
    for i in range(rb):
        st ^= (st << 13) & 0xFFFFFFFF
        st ^= st >> 17
        st ^= (st << 5) & 0xFFFFFFFF
        out[i] = st & 255
    if kind in (O.F32, O.BF16):
        for i in range(n):
            bits = np.float32((i % 127 - 63) / 64).view(np.uint32).item()
            if kind == O.F32:
                struct.pack_into("<I", out, 4 * i, bits)
            else:
                struct.pack_into("<H", out, 2 * i, bits >> 16)
    else:
        block, size, off = {O.Q8_0: (32, 34, 0), O.Q6_K: (256, 210, 208), O.IQ3_XXS: (256, 98, 0),
                            O.IQ4_NL: (32, 18, 0), O.IQ4_XS: (256, 136, 0)}[kind]
        for b in range(n // block):
            struct.pack_into("<H", out, b * size + off, [0x2000, 0x2800, 0x3000, 0xB000][b % 4])
    return np.frombuffer(bytes(out), np.uint8)


@pytest.mark.parametrize("kind", O.FRONTIER_KINDS)
def test_fixture_matches_python_restatement(kind):
    n = 2560
    assert np.array_equal(O.frontier_fixture(kind, n), py_fixture(kind, n))


@pytest.mark.parametrize("kind", O.FRONTIER_KINDS)
def test_linear_exact_sum_and_reference_tolerance(kind):
    n, m = 2560, 17
    raw = O.frontier_fixture(kind, n * m)
    x = ((np.arange(n) % 29 - 14) / 32).astype(np.float32)     # frontier_gpu.rs:95
    y = O.linear(kind, raw, n, m, x)
    W = O.dequantize(kind, raw, n * m).reshape(m, n).astype(np.float64)
    exact = (W * x.astype(np.float64)).sum(axis=1)             # products exact in float64
    assert np.array_equal(y, exact.astype(np.float32))
    seq = O.linear_f32seq(kind, raw, n, m, x)
    assert (np.abs(seq - y) <= 2e-4 + 2e-5 * np.abs(seq)).all()  # frontier_gpu.rs:111
