"""Pins the CPU oracle (oracle/uq_oracle.c) with closed forms, textbook float64
restatements, brute force and hand-built known-answer blocks.

The reference ships no golden vectors for this path (its checks are live
on-device gates: llm.rs:302-309, gpu_prefill.rs:95-121, gpu_graph.rs:14-23), so
each oracle function is checked against mathematics chosen so that a dropped
term, a wrong sign/index or a transposed operand fails.
"""
import numpy as np
import pytest

import oracle as O
import ggml_layouts as G

RNG = np.random.default_rng(1234)


def ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def rand_q8(rows, n, seed=7):
    rng = np.random.default_rng(seed)
    d = np.float16(rng.lognormal(np.log(0.01), 0.5, size=(rows, n // 32))).view(np.uint16)
    q = rng.integers(-127, 128, size=(rows, n), dtype=np.int64).astype(np.int8)
    return G.q8_0_pack(d, q)


# ---------------------------------------------------------------- fp16
def test_half_exhaustive_matches_ieee():
    O.lib()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([O.half(int(b)) for b in bits], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref))


def test_f16_rne_matches_numpy():
    specials = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 6.1e-5, 5.96e-8, 2.98e-8,
                         2.9802322e-08, 8.940697e-08, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, np.inf, -np.inf,
                         1e-30, 3.0e-5], np.float32)
    rnd = RNG.integers(0, 2 ** 32, size=200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    rnd = rnd[np.isfinite(rnd)]
    xs = np.concatenate([specials, rnd, RNG.normal(0, 30, 100000).astype(np.float32)])
    ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([O.f16_rne(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- exp
def lcg_samples(count):
    """The input stream of frontier_cpu_expf.rs:185-189: alternating dense
    decimal points in [-80, 80) and raw bit patterns with exponents < 133."""
    r, out = 17, []
    for i in range(count):
        r = (r * 1664525 + 1013904223) & 0xFFFFFFFF
        if i % 2 == 0:
            out.append(np.float32(((r % 160000) - 80000) / 1000.0))
        else:
            out.append(np.uint32((r & 0x807FFFFF) | (((r >> 24) % 133) << 23)).view(np.float32))
    return np.array(out, np.float32)


def test_expf_libm_algorithm_within_one_ulp():
    """uqo_expf restates libm 0.2.16 expf (frontier_cpu_expf.rs:80-170). It is
    not correctly rounded, so the check against float64 exp is <= 1 ulp; a
    dropped low-order reduction term or a wrong polynomial constant exceeds it
    (the lo term alone is k * 1.43e-6 relative, many ulps for k >= 1)."""
    xs = np.concatenate([np.linspace(-103.9, 88.7, 200001, dtype=np.float32),
                         RNG.uniform(-20, 20, 100000).astype(np.float32), lcg_samples(100000)])
    got = np.array([O.expf(float(x)) for x in xs], np.float32)
    ref = np.exp(xs.astype(np.float64)).astype(np.float32)
    d = ulp_diff(got, ref)
    assert d.max() <= 1
    assert (d == 0).mean() > 0.85


def test_expf_reduction_boundaries_and_specials():
    """Every branch boundary of the reduction (frontier_cpu_expf.rs:191-199):
    tiny |x| <= 2^-14 returns 1 + x, the +-1 reduction below 1.5 ln2, the
    multiple reduction, subnormal results below -87.34, zero from -103.97,
    overflow from 88.72."""
    for base in (0, 0x39000000, 0x3EB17218, 0x3F851592, 0x42A00000, 0x42AEAC50, 0x42B17218, 0x42CFF1B5):
        for dlt in range(-2, 3):
            for sign in (0, 0x80000000):
                bits = max(0, base + dlt) | sign
                x = np.uint32(bits).view(np.float32)
                got = np.float32(O.expf(float(x)))
                ref = np.float32(np.exp(np.float64(x)))
                if np.isinf(ref):
                    assert np.isinf(got) and got > 0, hex(bits)
                else:
                    assert ulp_diff(got, ref) <= 1, (hex(bits), got, ref)
    tiny = np.float32(2.0 ** -15)
    assert O.expf(float(tiny)) == np.float32(1) + tiny
    assert O.expf(0.0) == 1.0 and O.expf(-0.0) == 1.0
    assert O.expf(float(np.uint32(0x42CFF1B5 | 0x80000000).view(np.float32))) == 0.0
    assert O.expf(-200.0) == 0.0 and O.expf(200.0) == np.inf
    assert O.expf(float("inf")) == np.inf and O.expf(float("-inf")) == 0.0
    assert np.isnan(O.expf(float("nan")))
    sub = np.float32(O.expf(-95.0))                  # subnormal result
    assert 0 < sub < np.finfo(np.float32).tiny
    assert ulp_diff(sub, np.float32(np.exp(-95.0))) <= 1


# ---------------------------------------------------------------- activation quant
def test_quant_act_closed_form():
    x = RNG.normal(0, 1, 4096).astype(np.float32)
    x[0:32] = 0.0                                    # all-zero block
    x[32:64] = np.linspace(-3, 3, 32)
    x[64:96] = 1.0
    x[96] = -5.0                                     # negative amax
    q, s = O.quant_act(x)
    assert s[0] == 0 and not q[0:32].any()
    blocks = x.reshape(-1, 32)
    amax = np.abs(blocks).max(1)
    assert np.array_equal(s, (amax / np.float32(127)).astype(np.float32))
    qb = q.reshape(-1, 32).astype(np.int32)
    for b in range(1, blocks.shape[0]):
        j = np.argmax(np.abs(blocks[b]))
        assert abs(qb[b, j]) == 127 and np.sign(qb[b, j]) == np.sign(blocks[b, j])
    inv = np.where(amax > 0, np.float32(127) / amax, np.float32(0)).astype(np.float32)
    t = (blocks * inv[:, None]).astype(np.float32)
    assert np.array_equal(qb, np.clip(np.rint(t), -127, 127).astype(np.int32))  # np.rint: half to even
    err = np.abs(qb * s[:, None] - blocks)
    assert (err <= s[:, None] * 0.5 + 1e-6 * np.abs(blocks)).all()


def test_quant_act_ties_to_even():
    # amax 127 makes inv == 1 exactly, so x*inv hits the .5 ties directly
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5]
    q, s = O.quant_act(x)
    assert s[0] == np.float32(1.0)
    assert list(q[1:9]) == [0, 2, 2, 0, -2, -2, 4, 126]


# ---------------------------------------------------------------- Q8_0
def test_row_bytes_rules():
    # the reference's row_bytes gate (frontier_core.rs:53-58, its test :129-134)
    assert O.lib().uqo_row_bytes(O.Q8_0, 1536) == 1632
    assert O.lib().uqo_row_bytes(O.Q4_K, 1536) == 864
    assert O.lib().uqo_row_bytes(O.Q3_K, 256) == 110
    assert O.lib().uqo_row_bytes(O.F32, 3) == 12
    assert O.lib().uqo_row_bytes(O.Q4_K, 640) < 0
    assert O.lib().uqo_row_bytes(O.Q8_0, 0) < 0
    assert O.lib().uqo_row_bytes(99, 256) < 0


def test_q8_block_dots_brute_force():
    rows, n = 24, 256
    w = rand_q8(rows, n)
    qx = RNG.integers(-127, 128, n).astype(np.int8)
    dots = O.block_dots(O.Q8_0, w, n, rows, qx)
    _, q = G.q8_0_fields(w, rows, n)
    ref = (q.astype(np.int64) * qx.reshape(n // 32, 32).astype(np.int64)[None]).sum(-1)
    assert np.array_equal(dots, ref)


def test_q8_matvec_is_correctly_rounded_exact_sum():
    rows, n = 64, 1536
    w = rand_q8(rows, n)
    x = RNG.normal(0, 1, n).astype(np.float32)
    y = O.matvec(O.Q8_0, w, n, rows, x)
    qx, xs = O.quant_act(x)
    d, q = G.q8_0_fields(w, rows, n)
    c = (q.astype(np.int64) * qx.reshape(-1, 32).astype(np.int64)[None]).sum(-1)
    s = (G.f16_to_f32(d) * xs[None, :]).astype(np.float32)       # f32 product dw*dx
    terms = c.astype(np.float64) * s.astype(np.float64)           # exact in double
    from fractions import Fraction
    for r in range(0, rows, 7):                                   # exact rational sum, rounded once
        exact = sum(Fraction(float(t)) for t in terms[r])
        assert y[r] == np.float32(float(exact)) or ulp_diff(y[r], np.float32(float(exact))) <= 1
    ref = terms.sum(1).astype(np.float32)
    assert ulp_diff(y, ref).max() <= 1


def test_q8_matvec_vs_reference_literal_forms():
    rows, n = 40, 1536
    w = rand_q8(rows, n, seed=11)
    x = RNG.normal(0, 1, n).astype(np.float32)
    y = O.matvec(O.Q8_0, w, n, rows, x)
    lit = O.q8_matvec_f32seq(w, n, rows, x)        # gpu_prefill.rs:104-116 literal f32
    scale = np.abs(lit).max()
    assert (np.abs(y - lit) <= 1e-3 * np.maximum(np.abs(lit), 1e-3 * scale)).all()
    deq = O.q8_dequant_dot(w, n, rows, x)          # llm.rs:302-309 fp32 dequant dot
    dense = G.q8_0_dequant(w, rows, n).astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(deq, dense, rtol=1e-4, atol=1e-4 * np.abs(dense).max())
    # int8 activations vs fp32: the quantization error bound, not a bit match
    assert np.abs(y - dense).max() < 0.02 * np.abs(dense).max()


def test_q8_dequantize_matches_independent_layout():
    rows, n = 3, 256
    w = rand_q8(rows, n, seed=3)
    got = np.concatenate([O.dequantize(O.Q8_0, w[r * 272:(r + 1) * 272], n) for r in range(rows)])
    assert np.array_equal(got, G.q8_0_dequant(w, rows, n).reshape(-1))


# ---------------------------------------------------------------- Q4_K / Q3_K
def test_q4k_known_answer_block():
    # d = 1, dmin = 0, every sub-scale 1 -> value == q
    q = np.arange(256) % 16
    blk = G.q4_k_pack(0x3C00, 0x0000, [1] * 8, [0] * 8, q)
    assert np.array_equal(O.dequantize(O.Q4_K, blk, 256), q.astype(np.float32))
    # d = 0.5, dmin = 2, sc = j+1, m = 63-j (exercises the 6-bit high parts)
    sc, mn = [1, 17, 33, 49, 63, 5, 40, 62], [63, 2, 47, 16, 31, 60, 1, 33]
    blk = G.q4_k_pack(0x3800, 0x4000, sc, mn, q)
    d, dmin, sc2, mn2, q2 = G.q4_k_unpack(blk)
    assert list(sc2) == sc and list(mn2) == mn and np.array_equal(q2, q)
    exp = np.concatenate([np.float32(0.5 * sc[a]) * q[a * 32:(a + 1) * 32] - np.float32(2.0 * mn[a])
                          for a in range(8)]).astype(np.float32)
    assert np.array_equal(O.dequantize(O.Q4_K, blk, 256), exp)


def test_q3k_known_answer_block():
    q3 = np.arange(256) % 8
    scales = [32 + 1] * 16                       # (sc - 32) == 1
    blk = G.q3_k_pack(q3, scales, 0x3C00)        # d = 1 -> value == q3 - 4
    assert np.array_equal(O.dequantize(O.Q3_K, blk, 256), (q3 - 4).astype(np.float32))
    scales = list(range(0, 64, 4))               # 16 distinct 6-bit scales
    blk = G.q3_k_pack(q3[::-1].copy(), scales, 0x4000)
    vals, sc2, d = G.q3_k_unpack(blk)
    assert list(sc2) == scales and np.array_equal(vals, q3[::-1] - 4)
    exp = np.concatenate([np.float32(2.0 * (scales[k] - 32)) * (q3[::-1][16 * k:16 * (k + 1)] - 4)
                          for k in range(16)]).astype(np.float32)
    assert np.array_equal(O.dequantize(O.Q3_K, blk, 256), exp)


@pytest.mark.parametrize("kind", [O.Q4_K, O.Q3_K])
def test_kquant_dequant_matches_independent_layout(kind):
    rng = np.random.default_rng(kind)
    rows, n = 3, 512
    rb = 144 if kind == O.Q4_K else 110
    raw = rng.integers(0, 256, rows * (n // 256) * rb, dtype=np.int64).astype(np.uint8)
    # keep the fp16 scales finite and moderate
    blocks = raw.reshape(-1, rb)
    for off in ((0, 2) if kind == O.Q4_K else (108,)):
        blocks[:, off:off + 2] = np.float16(rng.uniform(0.001, 0.1, len(blocks))).view(np.uint8).reshape(-1, 2)
    got = np.stack([O.dequantize(kind, raw[r * (n // 256) * rb:(r + 1) * (n // 256) * rb], n) for r in range(rows)])
    ref = (G.q4_k_dequant if kind == O.Q4_K else G.q3_k_dequant)(raw, rows, n)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("kind", [O.Q4_K, O.Q3_K])
def test_kquant_integer_path_matches_dequant(kind):
    rng = np.random.default_rng(100 + kind)
    rows, n = 16, 768
    rb = 144 if kind == O.Q4_K else 110
    raw = rng.integers(0, 256, rows * (n // 256) * rb, dtype=np.int64).astype(np.uint8)
    blocks = raw.reshape(-1, rb)
    for off in ((0, 2) if kind == O.Q4_K else (108,)):
        blocks[:, off:off + 2] = np.float16(rng.uniform(0.001, 0.1, len(blocks))).view(np.uint8).reshape(-1, 2)
    x = rng.normal(0, 1, n).astype(np.float32)
    qx, xs = O.quant_act(x)
    y = O.matvec_q(kind, raw, n, rows, xs, qx)
    W = (G.q4_k_dequant if kind == O.Q4_K else G.q3_k_dequant)(raw, rows, n).astype(np.float64)
    xdq = (qx.reshape(-1, 32).astype(np.float64) * xs[:, None].astype(np.float64)).reshape(-1)
    ref = W @ xdq
    assert np.allclose(y, ref, rtol=2e-5, atol=2e-5 * np.abs(ref).max())
    # integer sums brute force
    dots = O.block_dots(kind, raw, n, rows, qx)
    if kind == O.Q4_K:
        qv = np.stack([G.q4_k_unpack(b)[4] for b in raw.reshape(-1, 144)]).reshape(rows, n)
        ref_d = (qv.reshape(rows, -1, 32) * qx.reshape(-1, 32)[None].astype(np.int64)).sum(-1)
    else:
        qv = np.stack([G.q3_k_unpack(b)[0] for b in raw.reshape(-1, 110)]).reshape(rows, n)
        ref_d = (qv.reshape(rows, -1, 16) * qx.reshape(-1, 16)[None].astype(np.int64)).sum(-1)
    assert np.array_equal(dots, ref_d)


# ---------------------------------------------------------------- prefill GEMM
def test_prefill_gemm_integer_and_bound():
    rows, n, batch = 48, 512, 9
    w = rand_q8(rows, n, seed=5)
    X = RNG.normal(0, 1, (batch, n)).astype(np.float32)
    qs = [O.quant_act(x) for x in X]
    qx = np.stack([a for a, _ in qs])
    xs = np.stack([b for _, b in qs])
    y = O.prefill_gemm(w, n, rows, xs, qx, batch)
    d, q = G.q8_0_fields(w, rows, n)
    c = np.einsum("rbk,tbk->trb", q.astype(np.int64), qx.reshape(batch, -1, 32).astype(np.int64))
    s = (G.f16_to_f32(d)[None] * xs[:, None, :]).astype(np.float32)
    ref = (c.astype(np.float64) * s.astype(np.float64)).sum(-1)
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
    # sequential fmaf order: a token's row equals the decode form to within rounding
    for t in range(batch):
        yd = O.matvec_q(O.Q8_0, w, n, rows, xs[t], qx[t])
        assert np.allclose(y[t], yd, rtol=1e-5, atol=1e-5 * np.abs(yd).max())
    # rows and tokens are independent: permuting tokens permutes outputs exactly
    perm = RNG.permutation(batch)
    y2 = O.prefill_gemm(w, n, rows, xs[perm], qx[perm], batch)
    assert np.array_equal(y2, y[perm])


# ---------------------------------------------------------------- norm / rope / attention / greedy
def test_rmsnorm_vs_float64():
    x = RNG.normal(0, 30, 1536).astype(np.float32)
    g = (1 + 0.1 * RNG.normal(0, 1, 1536)).astype(np.float32)
    y = O.rmsnorm(x, g)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean() + 1e-6) * g
    assert np.allclose(y, ref, rtol=3e-7 * 4, atol=0)
    assert np.allclose(O.rmsnorm(np.zeros(64, np.float32), np.ones(64, np.float32)), 0)


def test_rope_table_and_rotation():
    T = O.rope_table(640, 128, 1e6)
    assert np.array_equal(T[0, :64], np.ones(64, np.float32)) and np.array_equal(T[0, 64:], np.zeros(64, np.float32))
    pos = np.arange(640)[:, None].astype(np.float64)
    ang = pos * (1e6 ** (-(2 * np.arange(64)) / 128.0))[None]
    assert np.abs(T[:, :64] - np.cos(ang)).max() < 2e-4 and np.abs(T[:, 64:] - np.sin(ang)).max() < 2e-4
    v = RNG.normal(0, 5, 12 * 128).astype(np.float32)
    b = RNG.normal(0, 0.02, 12 * 128).astype(np.float32)
    assert np.array_equal(O.rope_bias(v, b, 12, 128, T[0]), (v + b).astype(np.float32))
    out = O.rope_bias(v, b, 12, 128, T[300])
    u = (v + b).astype(np.float64).reshape(12, 2, 64)
    c, s = T[300, :64].astype(np.float64), T[300, 64:].astype(np.float64)
    ref = np.stack([u[:, 0] * c - u[:, 1] * s, u[:, 0] * s + u[:, 1] * c], 1).reshape(-1)
    assert np.allclose(out, ref, rtol=1e-6, atol=1e-5)
    # rotation preserves each pair's norm
    o = out.astype(np.float64).reshape(12, 2, 64)
    assert np.allclose((o ** 2).sum(1), (u ** 2).sum(1), rtol=1e-5)


def test_attention_vs_float64_softmax():
    heads, kvh, hd, pos = 12, 2, 128, 200
    q = RNG.normal(0, 3, heads * hd).astype(np.float32)
    K = RNG.normal(0, 3, (pos + 1, kvh * hd)).astype(np.float16)
    V = RNG.normal(0, 3, (pos + 1, kvh * hd)).astype(np.float16)
    out = O.attention(q, K.view(np.uint16), V.view(np.uint16), pos, heads, kvh, hd)
    ref = np.zeros(heads * hd)
    for h in range(heads):
        kh = h // (heads // kvh)
        s = (K[:, kh * hd:(kh + 1) * hd].astype(np.float64) @ q[h * hd:(h + 1) * hd]) / np.sqrt(hd)
        pr = np.exp(s - s.max())
        pr /= pr.sum()
        ref[h * hd:(h + 1) * hd] = pr @ V[:, kh * hd:(kh + 1) * hd].astype(np.float64)
    assert np.allclose(out, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    # a single position returns v exactly (softmax of one element is exactly 1)
    out0 = O.attention(q, K.view(np.uint16), V.view(np.uint16), 0, heads, kvh, hd)
    v0 = V[0].astype(np.float32)
    assert np.array_equal(out0, np.concatenate([v0[(h // 6) * hd:(h // 6 + 1) * hd] for h in range(heads)]))


def test_greedy_tie_and_nonfinite_rules():
    x = RNG.normal(0, 1, 151936).astype(np.float32)
    i, bad = O.greedy(x)
    assert i == int(np.argmax(x)) and not bad
    x[10] = x[500] = x.max() + 1
    assert O.greedy(x) == (10, False)          # lowest id wins ties
    x[7] = np.nan
    assert O.greedy(x)[1]
    y = np.full(16, -np.inf, np.float32)
    assert O.greedy(y) == (0, True)


def test_silu_mul_vs_float64():
    g = np.concatenate([RNG.normal(0, 30, 2000), [0, -0.0, 100, -100, 88, -88]]).astype(np.float32)
    u = RNG.normal(0, 30, g.size).astype(np.float32)
    got = np.array([O.silu_mul(float(a), float(b)) for a, b in zip(g, u)], np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(got, ref, rtol=4e-7 * 4, atol=1e-30)


# ---------------------------------------------------------------- MoE routing
def test_moe_route_vs_stable_sort():
    for seed in range(20):
        lg = np.random.default_rng(seed).normal(0, 1, 128).astype(np.float32)
        if seed == 3:
            lg[5] = lg[77] = lg.max() + 0.5       # exact tie: lower id first
        rc, ids, w = O.moe_route(lg, 8)
        assert rc == 0
        p = np.exp(lg.astype(np.float64) - lg.max())
        p /= p.sum()
        order = sorted(range(128), key=lambda e: (-np.float32(p[e]), e))
        assert list(ids) == order[:8]
        assert np.allclose(w, p[ids] / p[ids].sum(), rtol=1e-6)
        assert abs(float(w.astype(np.float64).sum()) - 1) < 1e-6
    _, ids, _ = O.moe_route(np.zeros(128, np.float32), 8)
    assert list(ids) == list(range(8))


# ---------------------------------------------------------------- byte-literal K-quant known answers
# Literal superblocks written from ggml's published block structs and
# dequantize_row_q4_K / dequantize_row_q3_K (ggml-quants.c), independent of
# tests/ggml_layouts.py. Expected values are listed as 2*w (integers).
#
# Q4_K (block_q4_K: fp16 d, fp16 dmin, scales[12], qs[128]): d = 1.0, dmin =
# 0.5; 6-bit (scale, min) of the eight 32-value sub-blocks
# (3,9) (11,2) (7,12) (14,5) (17,44) (38,58) (53,6) (61,27): for j >= 4 the
# scale's high two bits sit in scales[j-4] >> 6 and the min's in scales[j] >> 6,
# and the two differ for every such j. qs[32k + l] holds sub-block 2k in its
# low nibble and 2k+1 in its high nibble; w = d*sc*q - dmin*m. The bytes are
# chosen so that swapping the two high-bit fields changes 128 of the 256
# values, and reading a byte's two nibbles as consecutive values changes 236.
Q4K_BLOCK = bytes.fromhex(
    "003c0038438bc7ce89c20c45c1a665bd00871e952ca33ab148cf56dd64eb72f9"
    "81089f16ad24bb32c940d75ee56cf37a35bc43ca51d86fe67df48b029910a72e"
    "b63dc44bd259e067fe750c831a9128af6ae178ff860d941ba229b037ce45dc53"
    "eb62f970078e159c23aa31b84fc65dd49f16ad24bb32c940d75ee56cf37a0188"
    "10972ea53cb34ac158df66ed74fb8209"
)
Q4K_2W = [
    -9, 33, 75, 21, 63, 9, 51, -3, 39, 81, 27, 69, 15, 57, 3, 45,
    -3, 39, 81, 27, 69, 15, 57, 3, 45, -9, 33, 75, 21, 63, 9, 51,
    -2, 174, 20, 196, 42, 218, 64, 240, 86, 262, 108, 284, 130, 306, 152, 328,
    174, -2, 196, 20, 218, 42, 240, 64, 262, 86, 284, 108, 306, 130, 328, 152,
    58, 156, 30, 128, 2, 100, 198, 72, 170, 44, 142, 16, 114, -12, 86, 184,
    72, 170, 44, 142, 16, 114, -12, 86, 184, 58, 156, 30, 128, 2, 100, 198,
    79, 303, 107, 331, 135, 359, 163, 387, 191, 415, 219, -5, 247, 23, 275, 51,
    303, 79, 331, 107, 359, 135, 387, 163, 415, 191, -5, 219, 23, 247, 51, 275,
    296, -10, 228, 466, 160, 398, 92, 330, 24, 262, -44, 194, 432, 126, 364, 58,
    330, 24, 262, -44, 194, 432, 126, 364, 58, 296, -10, 228, 466, 160, 398, 92,
    398, 1006, 474, 1082, 550, -58, 626, 18, 702, 94, 778, 170, 854, 246, 930, 322,
    1006, 398, 1082, 474, -58, 550, 18, 626, 94, 702, 170, 778, 246, 854, 322, 930,
    1584, 630, 1372, 418, 1160, 206, 948, -6, 736, 1478, 524, 1266, 312, 1054, 100, 842,
    -6, 736, 1478, 524, 1266, 312, 1054, 100, 842, 1584, 630, 1372, 418, 1160, 206, 948,
    1071, 95, 1193, 217, 1315, 339, 1437, 461, 1559, 583, 1681, 705, 1803, 827, -27, 949,
    95, 1071, 217, 1193, 339, 1315, 461, 1437, 583, 1559, 705, 1681, 827, 1803, 949, -27,
]

# Q3_K (block_q3_K: hmask[32], qs[64], scales[12], fp16 d): d = 0.5; the 16
# 6-bit scales 5 37 22 60 0 49 18 33 63 12 41 26 54 3 30 47 (value - 32 on
# decode), low four bits in scales[s] (s < 8) or scales[s-8] >> 4, high two
# bits in scales[8 + s%4] >> 2*(s/4). Value 128c + 32j + 16h + l reads bits
# 2j of qs[32c + 16h + l] and bit 4c+j of hmask[16h + l]; a clear hmask bit
# subtracts 4. The bytes are chosen so that an inverted hmask test changes
# all 256 values, taking the high bits from scales[8 + s/4] >> 2*(s%4)
# changes 112, and exchanging j and h for j < 2 changes 64.
Q3K_BLOCK = bytes.fromhex(
    "aa56a56a55a95a9595aa56a56a55a95a5a95aa56a56a55a9a95a95aa56a56a55"
    "500ffaa5500ffaa5a5500ffaa5500ffafaa5500ffaa5500f0ffaa5500ffaa550"
    "faa5500ffaa5500f0ffaa5500ffaa550500ffaa5500ffaa5a5500ffaa5500ffa"
    "f5c596ac6031e2f1f00e659b0038"
)
Q3K_2W = [
    108, 27, -54, 81, 0, -81, 54, -27, -27, 108, 27, -54, 81, 0, -81, 54,
    -10, 5, -20, -5, 10, -15, 0, 15, 15, -10, 5, -20, -5, 10, -15, 0,
    0, -30, 20, -10, 40, 10, -20, 30, 30, 0, -30, 20, -10, 40, 10, -20,
    56, -84, 0, 84, -56, 28, -112, -28, -28, 56, -84, 0, 84, -56, 28, -112,
    96, 0, -96, 64, -32, 128, 32, -64, -64, 96, 0, -96, 64, -32, 128, 32,
    -17, 34, -51, 0, 51, -34, 17, -68, -68, -17, 34, -51, 0, 51, -34, 17,
    -14, 56, 14, -28, 42, 0, -42, 28, 28, -14, 56, 14, -28, 42, 0, -42,
    3, -2, 1, -4, -1, 2, -3, 0, 0, 3, -2, 1, -4, -1, 2, -3,
    -62, 31, -124, -31, 62, -93, 0, 93, 93, -62, 31, -124, -31, 62, -93, 0,
    0, -60, 40, -20, 80, 20, -40, 60, 60, 0, -60, 40, -20, 80, 20, -40,
    18, -27, 0, 27, -18, 9, -36, -9, -9, 18, -27, 0, 27, -18, 9, -36,
    24, 6, -12, 18, 0, -18, 12, -6, -6, 24, 6, -12, 18, 0, -18, 12,
    -22, 44, -66, 0, 66, -44, 22, -88, -88, -22, 44, -66, 0, 66, -44, 22,
    -29, 116, 29, -58, 87, 0, -87, 58, 58, -29, 116, 29, -58, 87, 0, -87,
    -6, 4, -2, 8, 2, -4, 6, 0, 0, -6, 4, -2, 8, 2, -4, 6,
    -45, 0, 45, -30, 15, -60, -15, 30, 30, -45, 0, 45, -30, 15, -60, -15,
]


@pytest.mark.parametrize("kind,block,twice", [(O.Q4_K, Q4K_BLOCK, Q4K_2W), (O.Q3_K, Q3K_BLOCK, Q3K_2W)])
def test_kquant_byte_literal_known_answers(kind, block, twice):
    raw = np.frombuffer(block, np.uint8)
    assert raw.size == O.row_bytes(kind, 256)
    exp = (np.array(twice, np.float64) / 2).astype(np.float32)
    assert np.array_equal(O.dequantize(kind, raw, 256), exp)
    # the integer path sees the same codes: one-hot activations pick each value
    qx = np.zeros(256, np.int8)
    xs = np.ones(8, np.float32)
    for i in (0, 17, 31, 32, 63, 100, 127, 128, 200, 255):
        qx[:] = 0
        qx[i] = 1
        y = O.matvec_q(kind, raw, 256, 1, xs, qx)
        assert y[0] == exp[i], (i, y[0], exp[i])
