"""A Qwen2 model loaded from a GGUF file (uq_gguf_open + uq_model_load_gguf)
decodes like the oracle decoder over the same tensors (logits within 1 ulp,
identical greedy ids) and exactly like the same tensors set one by one
(uq_model_set_tensor): same logits bits, same ids. A file without
output.weight (tied embeddings) uses token_embd.weight as the output matrix.
A MoE layer read from a split model (uq_moe_load_gguf) matches the oracle's
Forward::ffn over the same expert bytes."""
import numpy as np
import pytest

import oracle as O
import uq
import gguf_writer as W


def ulps(a, b):
    a = a.view(np.int32).astype(np.int64)
    b = b.view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)

CFG = dict(layers=2, dim=256, hidden=512, heads=4, kv_heads=2, head_dim=64, vocab=1024, max_seq=128,
           eps=1e-6, theta=1e6)


@pytest.fixture(scope="module")
def gpu():
    uq.init(0)
    yield


def run(m, steps=12):
    first = m.decode_step(7, 0)
    logits = m.logits()
    ids, _ = m.decode_run(first, 1, steps)
    return first, logits, ids


@pytest.mark.gpu
@pytest.mark.parametrize("tie", [False, True])
def test_gguf_model_matches_direct_tensors(gpu, tmp_path, tie):
    tensors = uq.synth_qwen2(CFG, 0x5EED00AA)
    if tie:
        tensors["output.weight"] = tensors["token_embd.weight"]
    data, _ = W.qwen2_file(CFG, tensors, tie_output=tie)
    p = tmp_path / "qwen2.gguf"
    p.write_bytes(data)
    ref = uq.Qwen2Model(CFG, tensors)
    got = uq.Qwen2Model.from_gguf(str(p), CFG["max_seq"])
    f0, l0, i0 = run(ref)
    f1, l1, i1 = run(got)
    # the oracle decoder over the tensors the file holds (frontier_gguf.rs:86-137 reads them back by name)
    ora = O.Model(CFG, {k: v[3] for k, v in tensors.items()})
    rc, of, ol = ora.decode(7, 0, want_logits=True)
    assert rc == 0 and of == f1
    assert ulps(l1, ol).max() <= 1
    tok, oids = of, []
    for pos in range(1, 1 + len(i1)):
        rc, tok, _ = ora.decode(tok, pos)
        assert rc == 0
        oids.append(tok)
    assert list(i1) == oids
    assert f0 == f1
    assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32))
    assert np.array_equal(i0, i1)
    ref.free()
    got.free()


@pytest.mark.gpu
def test_gguf_model_rejects_unsupported_kinds(gpu, tmp_path):
    tensors = uq.synth_qwen2(CFG, 0x5EED00AB)
    kind, n, rows, arr = tensors["blk.0.ffn_up.weight"]
    # same bytes declared as Q4_K rows (144 B per 256 values): the dense decoder takes Q8_0 only
    raw = arr.tobytes()
    q4_rows = len(raw) // (n // 256 * 144)
    meta_cfg = dict(CFG)
    data, _ = W.write([("general.architecture", W.STRING, "qwen2")],
                      [("blk.0.ffn_up.weight", [n, q4_rows], 12, raw[:q4_rows * (n // 256 * 144)])])
    p = tmp_path / "bad.gguf"
    p.write_bytes(data)
    g = uq.Gguf.open(str(p))
    m = uq.Qwen2Model(meta_cfg)
    with pytest.raises(uq.UqError) as e:
        uq._check(uq.lib().uq_model_load_gguf(m.handle, g.handle))
    assert e.value.status == uq.Error.QUANT_TYPE
    m.free()
    g.free()


def moe_shards(cfg, seed, tmp_path, gate_inp=True):
    """A two-file split model of one MoE layer: shard 0 the shared expert (and
    its f32 gate), shard 1 the rank-3 expert banks [n, rows, experts]."""
    ex, sh, gi = uq.synth_moe(cfg, seed)
    D, F, E, k, sk = cfg["dim"], cfg["ff"], cfg["experts"], cfg["expert_kind"], cfg["shared_kind"]
    bank = lambda j: b"".join(e[j].tobytes() for e in ex)
    t0 = [("blk.0.ffn_gate_shexp.weight", [D, F], sk, sh[0].tobytes()),
          ("blk.0.ffn_up_shexp.weight", [D, F], sk, sh[1].tobytes()),
          ("blk.0.ffn_down_shexp.weight", [F, D], sk, sh[2].tobytes())]
    if gate_inp:
        t0.append(("blk.0.ffn_gate_inp_shexp.weight", [D], 0, gi.astype(np.float32).tobytes()))
    t1 = [("blk.0.ffn_gate_exps.weight", [D, F, E], k, bank(0)),
          ("blk.0.ffn_up_exps.weight", [D, F, E], k, bank(1)),
          ("blk.0.ffn_down_exps.weight", [F, D, E], k, bank(2))]
    total = len(t0) + len(t1)
    paths = []
    for no, ts in enumerate((t0, t1)):
        meta = [("split.no", W.U16, no), ("split.count", W.U16, 2), ("split.tensors.count", W.I32, total)]
        data, _ = W.write(meta, ts)
        p = tmp_path / ("moe-%05d-of-00002.gguf" % (no + 1))
        p.write_bytes(data)
        paths.append(str(p))
    return (ex, sh, gi if gate_inp else None), paths


@pytest.mark.gpu
@pytest.mark.parametrize("kind,gate_inp", [(uq.KIND_Q3_K, True), (uq.KIND_Q4_K, False)])
def test_moe_bank_from_split_gguf(gpu, tmp_path, kind, gate_inp):
    """uq_moe_load_gguf over a ModelIndex matches the oracle's Forward::ffn
    (frontier_forward.rs:164-199) over the same expert bytes: identical ids,
    bit-identical weights, outputs within 1 ulp; and it gives the same layer
    as uq_moe_set_expert / uq_moe_set_shared of those bytes, bit for bit."""
    cfg = dict(uq.MOE_CONFIG, dim=512, ff=256, experts=16, top_k=4, expert_kind=kind)
    (ex, sh, gi), paths = moe_shards(cfg, 0x5EED00C1 + kind, tmp_path, gate_inp)
    shards = [uq.Gguf.open(p) for p in reversed(paths)]
    ix = uq.GgufIndex(shards)
    a = uq.MoeLayer(cfg, ex, sh, gi)
    b = uq.MoeLayer.from_gguf(cfg, ix, 0)
    o = O.MoeLayer(cfg["dim"], cfg["ff"], cfg["experts"], cfg["top_k"], cfg["expert_kind"],
                   [e[0] for e in ex], [e[1] for e in ex], [e[2] for e in ex], cfg["shared_kind"],
                   sh[0], sh[1], sh[2], gi)
    try:
        for step in range(6):
            x = uq.synth_normal(0x5EED00C2 + 100 * step, cfg["dim"])
            lg = uq.synth_normal(0x5EED00C3 + 100 * step, cfg["experts"])
            oa, ia, wa = a.ffn(x, lg)
            ob, ib, wb = b.ffn(x, lg)
            rc, oo, io, wo = o.ffn(x, lg)
            assert rc == 0
            assert list(ib) == list(io), step
            assert np.array_equal(wb.view(np.uint32), wo.view(np.uint32))
            assert ulps(ob, oo).max() <= 1, step
            assert np.array_equal(ia, ib) and np.array_equal(wa.view(np.uint32), wb.view(np.uint32))
            assert np.array_equal(oa.view(np.uint32), ob.view(np.uint32))
    finally:
        a.free()
        b.free()
        ix.free()


@pytest.mark.gpu
def test_moe_load_rejects_wrong_shapes(gpu, tmp_path):
    cfg = dict(uq.MOE_CONFIG, dim=512, ff=256, experts=16, top_k=4)
    _, paths = moe_shards(cfg, 0x5EED00C4, tmp_path)
    ix = uq.GgufIndex([uq.Gguf.open(p) for p in paths])
    for bad, status in ((dict(cfg, experts=8), uq.Error.SHAPE), (dict(cfg, ff=512), uq.Error.SHAPE),
                        (dict(cfg, expert_kind=uq.KIND_Q4_K), uq.Error.QUANT_TYPE)):
        with pytest.raises(uq.UqError) as e:
            uq.MoeLayer.from_gguf(bad, ix, 0)
        assert e.value.status == status
    with pytest.raises(uq.UqError) as e:
        uq.MoeLayer.from_gguf(cfg, ix, 1)           # no blk.1 tensors
    assert e.value.status == uq.Error.FORMAT
    free, total = uq.device_memory()
    assert 0 < free <= total


@pytest.mark.gpu
def test_load_weight_whole_and_expert_slices(gpu, tmp_path):
    """uq_gguf_load_weight: a rank-2 tensor whole and the rows of single
    experts of a rank-3 frontier-kind tensor, each within 1 ulp of the oracle's
    exactly summed fp32-activation linear over the expert's rows
    (frontier_backend.rs:98-128 picks an expert's rows by offset), and equal
    (bit for bit, through uq_linear) to uploading those bytes directly."""
    n, rows, E = 512, 24, 3
    iq = uq.synth_quant(uq.KIND_IQ4_NL, 0x5EED00C5, rows * E, n)
    q8 = uq.synth_quant(uq.KIND_Q8_0, 0x5EED00C6, 40, n)
    data, _ = W.write([], [("blk.0.ffn_up_exps.weight", [n, rows, E], uq.KIND_IQ4_NL, iq.tobytes()),
                           ("blk.0.attn_q.weight", [n, 40], uq.KIND_Q8_0, q8.tobytes())])
    p = tmp_path / "w.gguf"
    p.write_bytes(data)
    g = uq.Gguf.open(str(p))
    x = uq.synth_normal(0x5EED00C7, n)
    ie, iw = g.find("blk.0.ffn_up_exps.weight"), g.find("blk.0.attn_q.weight")
    rb = uq.row_bytes(uq.KIND_IQ4_NL, n)
    for e in range(E):
        a = g.load_weight(ie, e)
        b = uq.Weight(uq.KIND_IQ4_NL, n, rows, iq[e * rows * rb:(e + 1) * rows * rb])
        ya = uq.linear(a, x)
        assert ulps(ya, O.linear(uq.KIND_IQ4_NL, iq[e * rows * rb:(e + 1) * rows * rb], n, rows, x)).max() <= 1
        assert np.array_equal(ya.view(np.uint32), uq.linear(b, x).view(np.uint32))
        a.free()
        b.free()
    a, b = g.load_weight(iw), uq.Weight(uq.KIND_Q8_0, n, 40, q8)
    ya = uq.linear(a, x)
    assert ulps(ya, O.linear(uq.KIND_Q8_0, q8, n, 40, x)).max() <= 1
    assert np.array_equal(ya.view(np.uint32), uq.linear(b, x).view(np.uint32))
    with pytest.raises(uq.UqError):
        g.load_weight(ie)                              # rank 3 needs an expert id
    with pytest.raises(uq.UqError):
        g.load_weight(ie, E)                           # no such expert
    g.free()
