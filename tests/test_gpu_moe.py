"""GPU MoE expert FFN (config: 128 Q3_K experts, top-8, dim 2048, ff 768, one
shared Q8_0 expert) against the oracle's Forward::ffn restatement, through the
C ABI: identical expert ids, bit-identical routing weights, outputs within 1
ulp (exact double sums rounded once on both sides)."""
import numpy as np
import pytest

import oracle as O
import uq

pytestmark = pytest.mark.gpu


def ulps(a, b):
    a = a.view(np.int32).astype(np.int64)
    b = b.view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def build(cfg, seed):
    ex, sh, gi = uq.synth_moe(cfg, seed)
    g = uq.MoeLayer(cfg, ex, sh, gi)
    o = O.MoeLayer(cfg["dim"], cfg["ff"], cfg["experts"], cfg["top_k"], cfg["expert_kind"],
                   [e[0] for e in ex], [e[1] for e in ex], [e[2] for e in ex], cfg["shared_kind"],
                   sh[0], sh[1], sh[2], gi)
    return g, o


# 128, 200 and 300 experts run the routing's rank with 4, 2 and 1 threads per expert
@pytest.mark.parametrize("cfg,steps", [(uq.MOE_CONFIG, 16),
                                       (dict(uq.MOE_CONFIG, dim=512, ff=256, experts=16, top_k=4), 8),
                                       (dict(uq.MOE_CONFIG, dim=512, ff=256, experts=200, top_k=8), 6),
                                       (dict(uq.MOE_CONFIG, dim=512, ff=256, experts=300, top_k=16), 6)])
def test_moe_matches_oracle(gpu, cfg, steps):
    g, o = build(cfg, 0x5EED0004)
    for step in range(steps):
        x = uq.synth_normal(0x5EED0004 + 1000 * step, cfg["dim"])
        lg = uq.synth_normal(0x5EED0004 + 1000 * step + 1, cfg["experts"])
        out, ids, w = g.ffn(x, lg)
        rc, oout, oids, ow = o.ffn(x, lg)
        assert rc == 0
        assert list(ids) == list(oids), step
        assert np.array_equal(w.view(np.uint32), ow.view(np.uint32))
        assert ulps(out, oout).max() <= 1, step


def test_moe_tie_and_nonfinite(gpu):
    cfg = dict(uq.MOE_CONFIG, dim=512, ff=256, experts=16, top_k=4)
    g, o = build(cfg, 7)
    x = uq.synth_normal(1, cfg["dim"])
    lg = np.zeros(cfg["experts"], np.float32)
    lg[3] = lg[9] = 2.0                      # tie: lower id first
    out, ids, w = g.ffn(x, lg)
    rc, oout, oids, ow = o.ffn(x, lg)
    assert list(ids) == list(oids) == [3, 9, 0, 1]
    assert ulps(out, oout).max() <= 1
    bad = lg.copy()
    bad[2] = np.nan
    with pytest.raises(uq.UqError) as e:
        g.ffn(x, bad)
    assert e.value.status == uq.Error.NONFINITE
    xb = x.copy()
    xb[0] = np.inf
    with pytest.raises(uq.UqError) as e:
        g.ffn(xb, lg)
    assert e.value.status == uq.Error.NONFINITE
