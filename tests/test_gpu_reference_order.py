"""GPU decode logits against the reference's own f32 operation orders.

The primary parity contract is bit-exact agreement with the exact-double
oracle (test_gpu_decode.py, test_gpu_golden.py). These tests compare the same
GPU runs, teacher-forced, with the oracle's reference-order decoder
(uqo_refo_*: the f32 orders of fused_resnorm, quant_act, qkv/gateup/linear
dp4a, rope_bias and fused_attention of the reference's decode graph,
gpu_graph.rs:137-162), with the KV cache in f32 as the reference keeps it and
rounded to fp16 as the library keeps it.

What is graded, and why: int8 activation quantization is discontinuous. A
last-ulp difference of two valid f32 orders occasionally moves one activation
code by one step; the random-init network then carries that change through
the residual stream and the cache, so logits of two orders differ by ~1e-3 to
~1e-2 of max|logit| at 2 layers and ~3% at 28 layers (the reference's own CPU
and GPU paths would differ alike). So the deviation is bounded at those
measured levels, and the greedy id must agree wherever the reference-order
top-2 margin exceeds twice the deviation observed at that step."""
import os

import numpy as np
import pytest

import oracle as O
import uq

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def dev(a, ref):
    return float(np.abs(a - ref).max() / np.abs(ref).max())


def margin(ref):
    s = np.sort(ref)
    return float((s[-1] - s[-2]) / np.abs(ref).max())


def test_two_layers_full_shape_teacher_forced(gpu):
    cfg = dict(uq.QWEN25_15B, layers=2, max_seq=128)
    t = uq.synth_qwen2(cfg, 0x5EED0002)
    arrays = {k: v[3] for k, v in t.items()}
    g = uq.Qwen2Model(cfg, t)
    refs = {"f16": O.RefoModel(cfg, arrays, kv_fp16=True), "f32": O.RefoModel(cfg, arrays, kv_fp16=False)}
    bound = {"f16": 2e-2, "f32": 0.15}
    toks = uq.synth_tokens(0x5EED0006, 64, cfg["vocab"])
    devs = {k: [] for k in refs}
    try:
        for pos, tok in enumerate(toks):
            nxt = g.decode_step(int(tok), pos)
            lg = g.logits()
            for k, r in refs.items():
                rc, rnext, rl = r.decode(int(tok), pos, want_logits=True)
                assert rc == 0
                d = dev(lg, rl)
                devs[k].append(d)
                assert d <= bound[k], (k, pos, d)
                if margin(rl) > 2 * d:
                    assert nxt == rnext, (k, pos, d, margin(rl))
    finally:
        g.free()
    print("median deviation: fp16 cache %.2e, f32 cache %.2e" % (np.median(devs["f16"]), np.median(devs["f32"])))


def test_28_layers_after_512_prompt_teacher_forced(gpu):
    """The 28-layer model of qwen25_decode.json: the GPU prefill of the
    512-token prompt, then all 128 decode steps fed the fixture's tokens (the
    build's own greedy ids, so the forced run is the free-running one),
    against tests/golden/qwen25_refo.npz (made by
    tests/golden/make_refo_golden.py): 129 positions, compared with the
    reference-order decoder with the KV cache in f32 and in fp16.

    Graded: the GPU's greedy ids equal the exact oracle's at every position;
    the logits stay within the measured deviation bound of the reference
    order; where the reference-order top-2 margin exceeds twice the step's
    deviation the ids agree; and the count of positions whose ids agree with
    the reference order is the fixture's (the exact oracle's) count."""
    import json
    g = json.load(open(os.path.join(HERE, "golden", "qwen25_decode.json")))
    f = np.load(os.path.join(HERE, "golden", "qwen25_refo.npz"))
    cfg = g["config"]
    m = uq.Qwen2Model(cfg, uq.synth_qwen2(cfg, g["seed"]))
    try:
        prompt = uq.synth_tokens(g["seed"], g["prompt_len"], cfg["vocab"])
        ids = [m.prefill(prompt)]
        logits = [m.logits()[f["idx"][0]]]
        for i, tok in enumerate(f["forced"]):
            ids.append(m.decode_step(int(tok), g["prompt_len"] + i))
            logits.append(m.logits()[f["idx"][i + 1]])
    finally:
        m.free()
    n = len(f["forced"]) + 1
    assert n == 129 and len(ids) == n
    assert ids[:-1] == [int(t) for t in f["forced"]]       # the fixture's tokens are the library's greedy ids
    assert ids == [int(t) for t in f["argmax_exact"]]      # and the exact oracle's, at all 129 positions
    # measured over the 129 positions (exact oracle vs reference order): fp16
    # cache max 0.047, median 0.028; f32 cache max 0.257, median 0.047
    for k, bound in (("f16", 0.06), ("f32", 0.3)):
        agree = 0
        for p, got in enumerate(logits):
            d = float(np.abs(got - f["ref_" + k][p]).max() / f["absmax_" + k][p])
            assert d <= bound, (k, p, d)
            if f["margin_" + k][p] / f["absmax_" + k][p] > 2 * d:
                assert ids[p] == int(f["argmax_" + k][p]), (k, p, d)
            agree += ids[p] == int(f["argmax_" + k][p])
        want = int((f["argmax_exact"] == f["argmax_" + k]).sum())
        assert agree == want, (k, agree, want)
        print("%s-cache reference order: greedy ids equal at %d of %d positions" % (k, agree, n))
