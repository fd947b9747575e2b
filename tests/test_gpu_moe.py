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


def orders(lg, top_k):
    """The oracle's exps and probabilities of these logits (exps with the
    oracle's expf after max subtraction, f32 running sum in expert order,
    p = e/sum): the top-k ids by (exp desc, id asc) and by (p desc, id asc)."""
    mx = np.float32(lg.max())
    e = np.array([O.expf(float(np.float32(v - mx))) for v in lg], np.float32)
    s = np.float32(0.0)
    for v in e:
        s = np.float32(s + v)
    p = (e / s).astype(np.float32)
    ids = np.arange(lg.size)
    by_e = [int(i) for i in sorted(ids, key=lambda i: (-e[i], i))[:top_k]]
    by_p = [int(i) for i in sorted(ids, key=lambda i: (-p[i], i))[:top_k]]
    return by_e, by_p


def collision_logits(experts, top_k, winners, seed):
    """Seeded logits with a cluster of experts whose logits are a few ulps
    apart (higher ids on the larger logits) near exp 0.9, `winners` clear
    leaders above them and the rest near -5 (sum of exps ~12): ulp-apart
    exps then round to equal probabilities about a third of the time. The
    first draw whose (p, id) top-k differs from the (exp, id) top-k."""
    rng = np.random.default_rng(seed)
    cluster = [10, 20, 30, 50, 60, 70]
    for _ in range(500):
        lg = rng.uniform(-5.5, -4.5, experts).astype(np.float32)
        for i, e in enumerate(range(40, 40 + winners)):
            lg[e] = np.float32(-0.01 * i)
        v = np.float32(-0.105 + rng.uniform(-0.01, 0.01))
        step = int(rng.integers(5, 25))
        for e in reversed(cluster):
            lg[e] = v
            for _ in range(step):
                v = np.nextafter(v, np.float32(-np.inf))
        by_e, by_p = orders(lg, top_k)
        if by_e != by_p:
            return lg, by_e, by_p
    raise AssertionError("no probability collision found")


# 6 leaders: the collision is at the top-k boundary and changes the set;
# 2 leaders: it is inside the top-k and changes the rank order only
@pytest.mark.parametrize("winners", [6, 2])
def test_moe_probability_collision(gpu, winners):
    """Experts whose exps differ by an ulp but whose probabilities round to the
    same value, lower ids on the smaller exps: the (p desc, id asc) order
    differs from the exp order, and the GPU must match the oracle's."""
    cfg = dict(uq.MOE_CONFIG, dim=512, ff=256, experts=128, top_k=8)
    g, o = build(cfg, 0x5EED00D1)
    x = uq.synth_normal(0x5EED00D2, cfg["dim"])
    lg, by_e, by_p = collision_logits(cfg["experts"], cfg["top_k"], winners, 0x5EED00D3 + winners)
    if winners == 6:
        assert set(by_e) != set(by_p)
    else:
        assert set(by_e) == set(by_p) and by_e != by_p
    out, ids, w = g.ffn(x, lg)
    rc, oout, oids, ow = o.ffn(x, lg)
    assert rc == 0
    assert list(oids) == by_p
    assert list(ids) == list(oids)
    assert np.array_equal(w.view(np.uint32), ow.view(np.uint32))
    assert ulps(out, oout).max() <= 1
