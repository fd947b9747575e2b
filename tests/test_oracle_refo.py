"""The reference-order decoder of the oracle (uqo_refo_*): the f32 operation
orders of the reference's decode-graph kernels. Each reduction order is pinned
by a hand-derived known answer whose inputs make the reference's order, an
exact sum and a plain sequential sum round to three different f32 values;
the rest is bounded against float64, and the whole decode against the exact
oracle."""
import numpy as np
import pytest

import oracle as O
import uq

F = np.float32


def q8_row(blocks, entries):
    """A Q8_0 row of `blocks` blocks: fp16 scale 1.0 everywhere, codes 0, then
    `entries` = {block: (fp16 bits, {byte index within the block: code})}."""
    row = np.zeros((blocks, 34), np.uint8)
    row[:, 0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    for b, (h, codes) in entries.items():
        row[b, 0:2] = np.frombuffer(np.uint16(h).tobytes(), np.uint8)
        for j, c in codes.items():
            row[b, 2 + j] = np.uint8(np.int8(c).view(np.uint8))
    return row.reshape(-1)


def test_resnorm_strided_tree_known_answer():
    # fused_resnorm (gpu_fused.cu:28-35): thread t sums the squares of x[t],
    # x[t+128], ...; the 128 sums meet in a tree of strides 64..1. x0 = 4096
    # (square 2^24) and ones at 1 + 128k and 2 + 128k, k = 0..10: s0 = 2^24,
    # s1 = s2 = 11. Stride 2: 2^24 + 11 -> 16777228 (tie to even); stride 1:
    # 16777228 + 11 -> 16777240. A sum in index order (the CPU norm of
    # llm.rs:323-327) drops every one: 2^24. The exact sum is 16777238.
    n = 1536
    x = np.zeros(n, F)
    x[0] = 4096
    for k in range(11):
        x[1 + 128 * k] = x[2 + 128 * k] = 1
    w = np.ones(n, F)
    _, y = O.refo_resnorm(x, np.zeros(n, F), w, eps=1e-6, add=False)

    def from_sum(s):
        mean = F(s) / F(n)
        scale = F(1) / np.sqrt(mean + F(1e-6))
        return (x * scale) * w

    assert np.array_equal(y, from_sum(16777240.0))
    assert not np.array_equal(y, from_sum(16777216.0))
    # the residual is added first and stored back
    r = np.arange(n, dtype=F) / F(n)
    xs, y2 = O.refo_resnorm(x, r, w, add=True)
    assert np.array_equal(xs, x + r)
    xr = (x + r).astype(np.float64)
    ref = xr / np.sqrt((xr * xr).mean() + 1e-6)
    assert np.allclose(y2, ref, rtol=2e-6, atol=1e-7)


def test_linear_dp4a_warp_combine_known_answer():
    # linear_dp4a (gpu_dp4a.cu:40-52) at K = 2048: thread t holds the 16-byte
    # half t&1 of block t>>1; warp w's butterfly total p_w covers blocks
    # 16w..16w+15 and the row is ((p0 + p1) + p2) + p3. p = (2^24, 1, 1, 2):
    # ((2^24 + 1) + 1) + 2 = 16777218; exact 16777220; pairwise 16777220.
    row = q8_row(64, {0: (0x6C00, {0: 64}), 16: (0x3C00, {0: 1}), 32: (0x3C00, {0: 1}), 48: (0x3C00, {0: 2})})
    qx = np.zeros(2048, np.int8)
    qx[[0, 512, 1024, 1536]] = [64, 1, 1, 1]
    xs = np.ones(64, F)
    assert O.refo_linear_row(row, xs, qx) == F(16777218.0)


def test_dotrow_lane_chain_and_butterfly_known_answer():
    # dotrow (gpu_dp4a.cu:32-39) at K = 2048: lane l takes bytes 8(l&3).. of
    # blocks l>>2, l>>2 + 8, ... in an fmaf chain, then the xor butterfly
    # 16, 8, 4, 2, 1. Lane 0: block 0 gives 2^24, block 8 gives 1, chained
    # fmaf(1, 1, 2^24) -> 2^24; lanes 8 and 24 (blocks 2 and 6) give 1 each
    # and meet first (xor 16), then join lane 0 (xor 8): 2^24 + 2 = 16777218.
    # Exact: 2^24 + 3 -> 16777220.
    row = q8_row(64, {0: (0x6C00, {0: 64}), 8: (0x3C00, {0: 1}), 2: (0x3C00, {0: 1}), 6: (0x3C00, {0: 1})})
    qx = np.zeros(2048, np.int8)
    qx[[0, 256, 64, 192]] = [64, 1, 1, 1]
    xs = np.ones(64, F)
    assert O.refo_dotrow(row, xs, qx) == F(16777218.0)


def test_attention_sequential_pv_known_answer():
    # fused_attention (gpu_attention.cu:2-26): zero keys give equal scores, so
    # p = 1/3 (f32) for T = 3, and out[i] = sum_t p_t v_t in t order. With v of
    # dim 0 = (3*2^24, 3, 3): p*3*2^24 -> 2^24, p*3 -> 1.0, and 2^24 + 1 + 1
    # stays 2^24 (ties to even). Exact: 2^24 + 2; reverse order: 2^24 + 2.
    hd, kvd, pos = 128, 256, 2
    q = np.linspace(-1, 1, hd).astype(F)
    keys = np.zeros((3, kvd), F)
    values = np.zeros((3, kvd), F)
    values[:, 0] = [3 * 2 ** 24, 3, 3]
    values[:, 5] = [1, 2, 3]
    out = O.refo_attention_head(q, keys, values, pos, 0, hd)
    assert out[0] == F(16777216.0)
    third = F(1) / F(3)
    assert out[5] == ((third * F(1)) + (third * F(2))) + (third * F(3))


def prefill_fmaf_case(blocks=4):
    """One Q8_0 row and one token whose per-block terms c_b * s_b are 2^24,
    3 * f32(1/3) = 1 + 2^-25, 1 (and 0 for a fourth block): the row's result
    separates the summation orders of a prefill GEMM row."""
    entries = {0: (0x3C00, {0: 1}), 1: (0x3C00, {0: 3}), 2: (0x3C00, {0: 1})}
    row = q8_row(blocks, entries)
    qx = np.zeros(32 * blocks, np.int8)
    qx[[0, 32, 64]] = 1
    xs = np.ones(blocks, F)
    xs[0] = F(2 ** 24)
    xs[1] = np.uint32(0x3EAAAAAB).view(F)
    return row, xs, qx


@pytest.mark.parametrize("blocks", [3, 4])
def test_prefill_gemm_sequential_fmaf_known_answer(blocks):
    # prefill_gemm (gpu_prefill.cu:10-36): f = fmaf((float)c_b, dw_b * dx_b, f)
    # for b = 0, 1, ... in order (lines 29-30). Terms 2^24, 1 + 2^-25, 1:
    #   fmaf chain:   2^24 -> rn(2^24 + 1 + 2^-25) = 2^24 + 2
    #                      -> rn(2^24 + 3) = 2^24 + 4 (tie to even)  = 16777220
    #   mul then add: rn(1 + 2^-25) = 1, 2^24 + 1 -> 2^24 twice     = 16777216
    #   fmaf, reversed block order: 1 -> rn(2 + 2^-25) = 2 -> 2^24 + 2 = 16777218
    #   exact sum 2^24 + 2 + 2^-25                                  -> 16777218
    row, xs, qx = prefill_fmaf_case(blocks)
    y = O.prefill_gemm(row, 32 * blocks, 1, xs[None], qx[None], 1)
    assert y[0, 0] == F(16777220.0)
    c = np.array([1, 3, 1, 0][:blocks], np.float64)
    terms = c * xs.astype(np.float64)                 # c_b * s_b, exact in double
    seq = F(0)
    mul_add = F(0)
    rev = F(0)
    for b in range(blocks):
        seq = F(np.float64(seq) + terms[b])           # one rounding of an exact double: fmaf
        mul_add = F(mul_add + F(terms[b]))
        rev = F(np.float64(rev) + terms[blocks - 1 - b])
    assert (seq, mul_add, rev) == (F(16777220.0), F(16777216.0), F(16777218.0))
    assert F(terms.sum()) == F(16777218.0)
    # the decode contract (exact double sum, rounded once) gives the exact form
    assert O.matvec_q(O.Q8_0, row, 32 * blocks, 1, xs, qx)[0] == F(16777218.0)


def test_attention_matches_float64():
    rng = np.random.default_rng(7)
    hd, kvd, pos = 128, 256, 300
    q = rng.normal(0, 1, hd).astype(F)
    keys = rng.normal(0, 1, (pos + 1, kvd)).astype(F)
    values = rng.normal(0, 1, (pos + 1, kvd)).astype(F)
    for kh in (0, 1):
        out = O.refo_attention_head(q, keys, values, pos, kh, hd)
        k = keys[:, kh * hd:(kh + 1) * hd].astype(np.float64)
        v = values[:, kh * hd:(kh + 1) * hd].astype(np.float64)
        s = k @ q.astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        ref = (p / p.sum()) @ v
        assert np.allclose(out, ref, rtol=1e-4, atol=2e-5)
        assert abs(float((p / p.sum()).sum()) - 1.0) < 1e-12


@pytest.mark.parametrize("K", [1536, 8960])
def test_dp4a_rows_match_exact_sum(K):
    raw = uq.synth_quant(uq.KIND_Q8_0, 0x5EED0001 + K, 24, K)
    x = uq.synth_normal(0x5EED0003 + K, K)
    qx, xs = O.quant_act(x)
    exact = O.matvec_q(O.Q8_0, raw, K, 24, xs, qx)
    rb = K // 32 * 34
    for r in range(24):
        row = raw[r * rb:(r + 1) * rb]
        for got in (O.refo_linear_row(row, xs, qx), O.refo_dotrow(row, xs, qx)):
            assert abs(got - exact[r]) <= 1e-5 * max(1.0, np.abs(exact).max())


SMALL = dict(layers=2, dim=256, hidden=512, heads=4, kv_heads=2, head_dim=64, vocab=1000, max_seq=64,
             eps=1e-6, theta=1e6)


@pytest.mark.parametrize("kv_fp16", [False, True])
def test_refo_decode_close_to_exact_oracle(kv_fp16):
    """The two decoders differ only in f32 order (and, with kv_fp16 False, the
    cache precision). Most steps agree to ~1e-7 of max|logit|; a last-ulp
    difference that moves one int8 activation code shows as an isolated
    jump, bounded here, and the greedy ids agree wherever the top-2 margin
    exceeds twice the step's deviation."""
    t = uq.synth_qwen2(SMALL, 0x5EED0002)
    arrays = {k: v[3] for k, v in t.items()}
    ex = O.Model(SMALL, arrays)
    rf = O.RefoModel(SMALL, arrays, kv_fp16=kv_fp16)
    toks = uq.synth_tokens(0x5EED0002, 20, SMALL["vocab"])
    devs = []
    for pos, tok in enumerate(toks):
        rc1, n1, l1 = ex.decode(int(tok), pos, want_logits=True)
        rc2, n2, l2 = rf.decode(int(tok), pos, want_logits=True)
        assert rc1 == 0 and rc2 == 0
        d = float(np.abs(l1 - l2).max() / np.abs(l2).max())
        devs.append(d)
        s = np.sort(l2)
        if (s[-1] - s[-2]) / np.abs(l2).max() > 2 * d:
            assert n1 == n2, pos
    # fp16 cache: order alone (isolated flips); f32 cache: the cache precision too
    assert max(devs) < (2e-2 if kv_fp16 else 6e-2) and np.median(devs) < (1e-5 if kv_fp16 else 3e-2), devs
