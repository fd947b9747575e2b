"""The Qwen2.5-1.5B-architecture greedy run against the committed oracle
fixture (tests/golden/qwen25_decode.json): random-init Q8_0 weights (seed
0x5EED0002), a 512-token seeded prompt through the GPU prefill, then 128
decode steps with the greedy id fed back on the device. Identical ids are
required (the fixture records the top-2 logit margins of each step)."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O
import uq

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def ulps(a, b):
    a = a.view(np.int32).astype(np.int64)
    b = b.view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


@pytest.fixture(scope="module")
def full_model(gpu):
    g = json.load(open(os.path.join(HERE, "golden", "qwen25_decode.json")))
    cfg = g["config"]
    t = uq.synth_qwen2(cfg, g["seed"])
    m = uq.Qwen2Model(cfg, t)
    yield g, cfg, t, m
    m.free()


def test_full_model_prefill_and_decode_match_golden(full_model):
    g, cfg, t, m = full_model
    prompt = uq.synth_tokens(g["seed"], g["prompt_len"], cfg["vocab"])
    assert hashlib.sha256(prompt.tobytes()).hexdigest() == g["prompt_sha256"]
    first = m.prefill(prompt)
    assert first == g["first_id"]
    ids, _ = m.decode_run(first, g["prompt_len"], g["steps"])
    assert [int(i) for i in ids] == g["ids"]


@pytest.mark.parametrize("layers,n", [(28, 48), (4, 512)])
def test_prefill_depth_and_length(gpu, layers, n):
    cfg = dict(uq.QWEN25_15B, layers=layers, max_seq=1024)
    t = uq.synth_qwen2(cfg, 0x5EED0002)
    gm = uq.Qwen2Model(cfg, t)
    toks = uq.synth_tokens(0x5EED0002, n, cfg["vocab"])
    nxt = gm.prefill(toks)
    lg = gm.logits()
    k, v = gm.kv(layers - 1, n)
    gm.free()
    O.set_threads(16)
    om = O.Model(cfg, {kk: vv[3] for kk, vv in t.items()})
    rc, onxt, olg = om.prefill(toks, want_logits=True)
    assert rc == 0
    ok = om.keys(layers - 1, n)
    bad_rows = np.nonzero((k != ok).any(1))[0]
    assert bad_rows.size == 0, ("first differing key position", int(bad_rows[0]))
    assert np.array_equal(v, om.values(layers - 1, n))
    assert ulps(lg, olg).max() <= 1
    assert nxt == onxt
