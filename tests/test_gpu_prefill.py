"""GPU prefill (int8 MFMA GEMM + batched norm/RoPE/attention) against the
oracle, through the C ABI. The GEMM keeps the reference's sequential per-block
fmaf update (gpu_prefill.cu:29-30), so outputs are compared bit for bit; the
int32 block dots inside it are exact by construction of that comparison."""
import numpy as np
import pytest

import oracle as O
import uq

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, dim=256, hidden=512, heads=4, kv_heads=2, head_dim=64, vocab=1000, max_seq=128,
             eps=1e-6, theta=1e6)


def ulps(a, b):
    a = a.view(np.int32).astype(np.int64)
    b = b.view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def quant_rows(X):
    qs = [O.quant_act(x) for x in X]
    return np.stack([q for q, _ in qs]), np.stack([s for _, s in qs])


# (4096, 1536, 512) and (4096, 1568, 512) run the 32 x 64 workgroup tiles;
# the others give grids of under four workgroups per CU and run the 32 x 32
# tiles (1536 and 2048 rows at 450-512 tokens: the model's o, down and fused
# q,k,v shapes). A stage holds 4 blocks (K 128): K 160 is one full stage and
# a partial one, 384 an odd count of full stages (the last one after the
# paired loop), 416 three full stages and a partial one, 1568 twelve and a
# partial one.
@pytest.mark.parametrize("N,K,T", [(1536, 1536, 512), (256, 1536, 77), (8960, 1536, 64), (1536, 8960, 40),
                                   (64, 32, 1), (128, 64, 130), (4096, 1536, 512),
                                   (64, 160, 33), (128, 384, 70), (64, 416, 64), (4096, 1568, 512),
                                   (1536, 1568, 512), (1536, 384, 500), (2048, 1536, 512), (2048, 416, 512),
                                   (2048, 160, 450)])
def test_prefill_gemm_bit_exact(gpu, N, K, T):
    raw = uq.synth_quant(uq.KIND_Q8_0, 0x5EED0003 + N, N, K)
    X = np.stack([uq.synth_normal(0x5EED0003 + t, K) for t in range(T)])
    qx, xs = quant_rows(X)
    w = uq.Weight(uq.KIND_Q8_0, K, N, raw)
    y = uq.prefill_gemm(w, qx, xs)
    ref = O.prefill_gemm(raw, K, N, xs, qx, T)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), ulps(y, ref).max()


# Token rows whose activation scales make dw * dx subnormal (x ~ 1e-35: dx ~
# 2e-37, dw ~ 1e-2), zero, or large (x ~ 1e25), beside ordinary rows; the
# scale product must be the f32 multiply with denormals kept on both the
# outer-product MFMA path (full stages) and the VALU path (partial stage).
@pytest.mark.parametrize("N,K,T", [(128, 1536, 64), (128, 416, 64), (128, 96, 64), (1536, 1536, 512),
                                   (2048, 416, 512)])
def test_prefill_gemm_extreme_scales(gpu, N, K, T):
    raw = uq.synth_quant(uq.KIND_Q8_0, 0x5EED00E0 + K, N, K)
    mags = [1.0, 1e-35, 0.0, 1e25, 3e-33, 1e-36, 1e20, 1e-30]
    X = np.stack([uq.synth_normal(0x5EED00E1 + t, K) * np.float32(mags[t % len(mags)]) for t in range(T)])
    X = X.astype(np.float32)
    qx, xs = quant_rows(X)
    assert (xs[1::8] * 0.02 < np.finfo(np.float32).tiny).all()        # subnormal scale products
    w = uq.Weight(uq.KIND_Q8_0, K, N, raw)
    y = uq.prefill_gemm(w, qx, xs)
    ref = O.prefill_gemm(raw, K, N, xs, qx, T)
    assert np.isfinite(ref).all() and (ref[2::8] == 0).all() and (np.abs(ref[1::8]) > 0).any()
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), ulps(y, ref).max()


@pytest.mark.parametrize("blocks,N,T", [(3, 64, 2), (4, 64, 2), (3, 1536, 512), (8, 2048, 512)])
def test_prefill_gemm_sequential_fmaf_known_answer(gpu, blocks, N, T):
    """Row 0 of the weight and token 0 give per-block terms 2^24, 1 + 2^-25,
    1 (then 0): the reference's in-order fmaf chain (gpu_prefill.cu:29-30)
    rounds to 16777220, a multiply-then-add chain to 16777216 and the reversed
    block order or the exact sum to 16777218. K 96 runs the partial-stage path,
    K 128 one full stage; N 1536 / 2048 at 512 tokens the model's launch
    shapes."""
    K = 32 * blocks
    raw = uq.synth_quant(uq.KIND_Q8_0, 0x5EED00E2, N, K).copy()
    rb = K // 32 * 34
    row = np.zeros((blocks, 34), np.uint8)
    row[:, 0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    row[0, 2], row[1, 2], row[2, 2] = 1, 3, 1
    raw[:rb] = row.reshape(-1)
    qx = np.zeros((T, K), np.int8)
    xs = np.ones((T, blocks), np.float32)
    qx[0, [0, 32, 64]] = 1
    xs[0, 0] = 2.0 ** 24
    xs[0, 1] = np.uint32(0x3EAAAAAB).view(np.float32)
    for t in range(1, T):
        qx[t], xs[t] = O.quant_act(uq.synth_normal(0x5EED00E3 + t, K))
    w = uq.Weight(uq.KIND_Q8_0, K, N, raw)
    y = uq.prefill_gemm(w, qx, xs)
    assert y[0, 0] == np.float32(16777220.0)
    ref = O.prefill_gemm(raw, K, N, xs, qx, T)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), ulps(y, ref).max()


def build(cfg, seed):
    t = uq.synth_qwen2(cfg, seed)
    return uq.Qwen2Model(cfg, t), O.Model(cfg, {k: v[3] for k, v in t.items()})


@pytest.mark.parametrize("n", [1, 7, 64, 100])
def test_prefill_matches_oracle(gpu, n):
    g, o = build(SMALL, 21)
    toks = uq.synth_tokens(21 + n, n, SMALL["vocab"])
    nxt = g.prefill(toks)
    rc, onxt, olg = o.prefill(toks, want_logits=True)
    assert rc == 0
    assert ulps(g.logits(), olg).max() <= 1
    assert nxt == onxt
    for layer in range(SMALL["layers"]):
        k, v = g.kv(layer, n)
        assert np.array_equal(k, o.keys(layer, n)) and np.array_equal(v, o.values(layer, n))


# KV capacities that are not a multiple of the 64-token GEMM tile: the prompt
# fills the cache to its last position, so every attention key read must stay
# inside [0, n) of the allocation
@pytest.mark.parametrize("max_seq,n", [(100, 100), (97, 97), (97, 50), (65, 65)])
def test_prefill_kv_capacity_not_tile_multiple(gpu, max_seq, n):
    cfg = dict(SMALL, max_seq=max_seq)
    g, o = build(cfg, 57)
    toks = uq.synth_tokens(57 + n, n, cfg["vocab"])
    nxt = g.prefill(toks)
    rc, onxt, olg = o.prefill(toks, want_logits=True)
    assert rc == 0 and nxt == onxt
    assert ulps(g.logits(), olg).max() <= 1
    for layer in range(cfg["layers"]):
        k, v = g.kv(layer, n)
        assert np.array_equal(k, o.keys(layer, n)) and np.array_equal(v, o.values(layer, n))


# models without some or all of the q/k/v biases (the prefill's fused RoPE
# epilogue and decode's qkv kernel then add nothing: x + 0.0 would turn -0.0
# into +0.0)
@pytest.mark.parametrize("drop", [("attn_q.bias", "attn_k.bias", "attn_v.bias"), ("attn_k.bias",)])
def test_prefill_and_decode_without_biases(gpu, drop):
    t = {k: v for k, v in uq.synth_qwen2(SMALL, 91).items() if not k.endswith(drop)}
    g, o = uq.Qwen2Model(SMALL, t), O.Model(SMALL, {k: v[3] for k, v in t.items()})
    toks = uq.synth_tokens(91, 70, SMALL["vocab"])
    first = g.prefill(toks)
    rc, ofirst, olg = o.prefill(toks, want_logits=True)
    assert rc == 0 and first == ofirst
    assert ulps(g.logits(), olg).max() <= 1
    for layer in range(SMALL["layers"]):
        k, v = g.kv(layer, 70)
        assert np.array_equal(k, o.keys(layer, 70)) and np.array_equal(v, o.values(layer, 70))
    ids, _ = g.decode_run(first, 70, 12)
    tok, ref = ofirst, []
    for pos in range(70, 82):
        rc, tok, _ = o.decode(tok, pos)
        assert rc == 0
        ref.append(tok)
    assert list(ids) == ref


def test_prefill_then_decode(gpu):
    g, o = build(SMALL, 33)
    toks = uq.synth_tokens(33, 50, SMALL["vocab"])
    first = g.prefill(toks)
    rc, ofirst, _ = o.prefill(toks)
    assert rc == 0 and first == ofirst
    ids, _ = g.decode_run(first, 50, 30)
    tok, ref = ofirst, []
    for pos in range(50, 80):
        rc, tok, _ = o.decode(tok, pos)
        assert rc == 0
        ref.append(tok)
    assert list(ids) == ref


def test_prefill_qwen25_shapes_two_layers(gpu):
    cfg = dict(uq.QWEN25_15B, layers=2, max_seq=256)
    g, o = build(cfg, 0x5EED0002)
    toks = uq.synth_tokens(0x5EED0002, 96, cfg["vocab"])
    nxt = g.prefill(toks)
    rc, onxt, olg = o.prefill(toks, want_logits=True)
    assert rc == 0 and nxt == onxt
    assert ulps(g.logits(), olg).max() <= 1


def test_prefill_rejects_bad_input(gpu):
    g, _ = build(SMALL, 4)
    with pytest.raises(uq.UqError) as e:
        g.prefill(np.array([SMALL["vocab"]], np.uint32))
    assert e.value.status == uq.Error.SHAPE
    with pytest.raises(uq.UqError) as e:
        g.prefill(np.zeros(SMALL["max_seq"] + 1, np.uint32))
    assert e.value.status == uq.Error.CONTEXT
