"""GPU decode step (hipGraph) against the oracle decoder, through the C ABI.

Every reduction on both sides accumulates exactly formed terms in double and
rounds once, so logits, KV cache contents and greedy ids are expected to agree
bit for bit; the assertions allow at most 1 ulp on logits (rounding of a sum
that lands within 2^-29 of a tie) and require identical greedy ids."""
import numpy as np
import pytest

import oracle as O
import uq

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, dim=256, hidden=512, heads=4, kv_heads=2, head_dim=64, vocab=1000, max_seq=64,
             eps=1e-6, theta=1e6)


def ulps(a, b):
    a = a.view(np.int32).astype(np.int64)
    b = b.view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def build(cfg, seed):
    t = uq.synth_qwen2(cfg, seed)
    gpu = uq.Qwen2Model(cfg, t)
    ora = O.Model(cfg, {k: v[3] for k, v in t.items()})
    return gpu, ora


@pytest.mark.parametrize("cfg,steps", [(SMALL, 24), (dict(SMALL, layers=3, dim=512, hidden=1024, heads=8,
                                                          kv_heads=2, head_dim=64, vocab=3000), 12),
                                       (dict(SMALL, max_seq=4096), 24)])   # a long cache: attention LDS sized to max_seq
def test_decode_steps_teacher_forced(gpu, cfg, steps):
    g, o = build(cfg, 0x5EED0002)
    toks = uq.synth_tokens(0x5EED0002, steps, cfg["vocab"])
    for pos in range(steps):
        nxt = g.decode_step(int(toks[pos]), pos)
        lg = g.logits()
        rc, onxt, olg = o.decode(int(toks[pos]), pos, want_logits=True)
        assert rc == 0
        d = ulps(lg, olg)
        assert d.max() <= 1, (pos, d.max(), (d > 0).sum())
        assert nxt == onxt, pos
    for layer in range(cfg["layers"]):
        k, v = g.kv(layer, steps)
        assert np.array_equal(k, o.keys(layer, steps)) and np.array_equal(v, o.values(layer, steps))


def test_decode_run_free_running(gpu):
    g, o = build(SMALL, 77)
    first = 17
    out, ms = g.decode_run(first, 0, 40)
    tok, ref = first, []
    for pos in range(40):
        rc, tok, _ = o.decode(tok, pos)
        assert rc == 0
        ref.append(tok)
    assert list(out) == ref
    assert ms > 0


def test_decode_rejects_bad_position_and_token(gpu):
    g, _ = build(SMALL, 5)
    with pytest.raises(uq.UqError) as e:
        g.decode_step(3, SMALL["max_seq"])
    assert e.value.status == uq.Error.CONTEXT
    with pytest.raises(uq.UqError) as e:
        g.decode_step(SMALL["vocab"], 0)
    assert e.value.status == uq.Error.SHAPE
    with pytest.raises(uq.UqError) as e:
        g.decode_run(1, SMALL["max_seq"] - 4, 8)
    assert e.value.status == uq.Error.CONTEXT


def test_model_requires_every_tensor(gpu):
    t = uq.synth_qwen2(SMALL, 3)
    m = uq.Qwen2Model(SMALL)
    for name, (kind, n, rows, arr) in t.items():
        if name != "blk.1.ffn_down.weight":
            m.set_tensor(name, kind, n, rows, arr)
    with pytest.raises(uq.UqError) as e:
        m.prepare()
    assert "blk.1.ffn_down.weight" in str(e.value)
    raw = t["blk.1.ffn_down.weight"][3]
    with pytest.raises(uq.UqError) as e:                       # byte count != rows * row_bytes
        m.set_tensor("blk.1.ffn_down.weight", uq.KIND_Q8_0, 512, 256, raw[:-34])
    assert e.value.status == uq.Error.SHAPE
    m.set_tensor("blk.1.ffn_down.weight", uq.KIND_Q8_0, 256, 512, raw)   # transposed shape
    with pytest.raises(uq.UqError) as e:
        m.prepare()
    assert e.value.status == uq.Error.SHAPE and "ffn_down" in str(e.value)
    m.set_tensor("blk.1.ffn_down.weight", uq.KIND_Q8_0, 512, 256, raw)
    m.prepare()
    assert m.decode_step(1, 0) < SMALL["vocab"]


def test_decode_qwen25_shapes_two_layers(gpu):
    """The real Qwen2.5-1.5B shapes (dim 1536, ffn 8960, 12/2 heads of 128,
    vocab 151936) with two layers, against the oracle step by step."""
    cfg = dict(uq.QWEN25_15B, layers=2, max_seq=64)
    g, o = build(cfg, 0x5EED0002)
    toks = uq.synth_tokens(9, 6, cfg["vocab"])
    for pos in range(6):
        nxt = g.decode_step(int(toks[pos]), pos)
        rc, onxt, olg = o.decode(int(toks[pos]), pos, want_logits=True)
        assert rc == 0 and nxt == onxt
        assert ulps(g.logits(), olg).max() <= 1


def _replace(tensors, name, raw):
    kind, n, rows, _ = tensors[name]
    out = dict(tensors)
    out[name] = (kind, n, rows, raw)
    return out


@pytest.mark.parametrize("cfg", [SMALL, dict(uq.QWEN25_15B, layers=1, max_seq=64)])
def test_greedy_tie_takes_lowest_id(gpu, cfg):
    """Two byte-identical lm_head rows give bit-identical logits; the greedy id
    is the lower of the two (gpu_greedy.cu:1-27, gpu_graph.rs:14-23), whether
    the twin row sits in the same argmax workgroup or in another one."""
    t = uq.synth_qwen2(cfg, 41)
    o = O.Model(cfg, {k: v[3] for k, v in t.items()})
    rc, a, olg = o.decode(5, 0, want_logits=True)
    assert rc == 0 and (olg == olg[a]).sum() == 1          # a unique maximum to start from
    rb = cfg["dim"] // 32 * 34
    vocab = cfg["vocab"]
    for b in sorted({a - 1, a + 1, 0, vocab - 1} - {a}):
        if not 0 <= b < vocab:
            continue
        raw = t["output.weight"][3].copy()
        raw[b * rb:(b + 1) * rb] = raw[a * rb:(a + 1) * rb]
        t2 = _replace(t, "output.weight", raw)
        g = uq.Qwen2Model(cfg, t2)
        try:
            nxt = g.decode_step(5, 0)
            lg = g.logits()
            assert lg[a].view(np.uint32) == lg[b].view(np.uint32)
            assert nxt == min(a, b), (a, b, nxt)
            o2 = O.Model(cfg, {k: v[3] for k, v in t2.items()})
            assert o2.decode(5, 0)[1] == min(a, b)
            # the tie survives into the device-fed loop: the second step starts from min(a, b)
            ids, _ = g.decode_run(5, 0, 2)
            assert ids[0] == min(a, b) and ids[1] == o2.decode(min(a, b), 1)[1]
        finally:
            g.free()


def test_nonfinite_logit_fails_the_step(gpu):
    """One fp16 NaN (then +inf) scale in one lm_head row: that logit is
    non-finite and every greedy entry point returns UQ_ERR_NONFINITE (the bad
    flag of gpu_greedy.cu:1-27). An infinite output-norm weight makes one
    activation infinite: its block quantizes to codes 0 with scale inf, and
    0 * inf makes every logit NaN. The run still fails with NONFINITE, and the
    id fed back on the device between steps stays inside the vocabulary."""
    t = uq.synth_qwen2(SMALL, 43)
    rb = SMALL["dim"] // 32 * 34
    toks = uq.synth_tokens(43, 9, SMALL["vocab"])
    for scale in (b"\x00\x7e", b"\x00\x7c"):          # fp16 0x7E00 NaN, 0x7C00 +inf (little endian)
        raw = t["output.weight"][3].copy()
        row = 123
        raw[row * rb + 34 * 2:row * rb + 34 * 2 + 2] = np.frombuffer(scale, np.uint8)   # block 2 of row 123
        g = uq.Qwen2Model(SMALL, _replace(t, "output.weight", raw))
        try:
            for call in (lambda: g.decode_step(5, 0), lambda: g.decode_run(5, 0, 3), lambda: g.prefill(toks)):
                with pytest.raises(uq.UqError) as e:
                    call()
                assert e.value.status == uq.Error.NONFINITE
            assert not np.isfinite(g.logits()[row])
        finally:
            g.free()
    gamma = t["output_norm.weight"][3].copy()
    gamma[7] = np.inf
    g = uq.Qwen2Model(SMALL, _replace(t, "output_norm.weight", gamma))
    try:
        with pytest.raises(uq.UqError) as e:
            g.decode_run(5, 0, 4)
        assert e.value.status == uq.Error.NONFINITE
        assert np.isnan(g.logits()).all()
        with pytest.raises(uq.UqError) as e:
            g.decode_step(5, 4)
        assert e.value.status == uq.Error.NONFINITE
    finally:
        g.free()
