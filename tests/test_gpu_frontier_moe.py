"""The frontier MoE block (Forward::ffn, driver/src/frontier_forward.rs:164-199)
composed on the fp32-activation reader: the router as one uq_linear, then the
two Weights::batch job tables (10 routed experts' gate and up, the shared
expert's gate and up and its 1-row scale; then the 11 down projections) as two
uq_linear_batch launches, with the reference's host arithmetic between them
(softmax, stable top-10, SiLU, sigmoid, rank-ordered mul-then-add).

The same host arithmetic over the oracle's linears (uqo_linear) is the
reference side; the block output must agree to 1e-3 of its max-norm and the
routed ids exactly. Kinds follow the reference's expert probe
(frontier_gpu.rs:245-278): IQ3_XXS gate/up, IQ4_NL down, F32 router."""
import numpy as np
import pytest

import oracle as O
import uq

pytestmark = pytest.mark.gpu

D, FF, E, K = 2560, 640, 64, 10


def expf(v):
    return np.array([O.expf(float(t)) for t in np.ravel(v)], np.float32).reshape(np.shape(v))


def sigmoid(v):
    one = np.float32(1.0)
    return (one / (one + expf(-np.asarray(v, np.float32)))).astype(np.float32)


def softmax(x):
    """frontier_forward.rs:47-51: max subtraction, f32 running sum, divide."""
    x = np.asarray(x, np.float32)
    e = expf(x - np.float32(x.max()))
    s = np.float32(0.0)
    for v in e:
        s = np.float32(s + v)
    return (e / s).astype(np.float32)


def ffn(linear, batch, W, x):
    """Forward::ffn with `linear(key, x)` and `batch([(key, x), ...])`."""
    scores = softmax(linear(("router", None), x))
    ids = sorted(range(E), key=lambda i: (-scores[i], i))[:K]
    tot = np.float32(0.0)
    for i in ids:
        tot = np.float32(tot + scores[i])
    reqs = []
    for e in ids:
        reqs += [(("gate", e), x), (("up", e), x)]
    reqs += [(("sgate", None), x), (("sup", None), x), (("sscale", None), x)]
    proj = batch(reqs)
    assert len(proj) == 23 and all(len(v) == FF for v in proj[:22]) and len(proj[22]) == 1
    middle = [(proj[2 * i] * sigmoid(proj[2 * i])).astype(np.float32) * proj[2 * i + 1] for i in range(11)]
    middle = [m.astype(np.float32) for m in middle]
    reqs = [(("down", e), middle[i]) for i, e in enumerate(ids)] + [(("sdown", None), middle[10])]
    vals = batch(reqs)
    out = np.zeros(D, np.float32)
    for r, e in enumerate(ids):
        w = np.float32(scores[e] / tot)
        out = (out + (w * vals[r]).astype(np.float32)).astype(np.float32)
    w = sigmoid(proj[22][0])
    out = (out + (w * vals[10]).astype(np.float32)).astype(np.float32)
    return out, ids


@pytest.fixture(scope="module")
def bank(gpu):
    specs = {("router", None): (uq.KIND_F32, D, E), ("sscale", None): (uq.KIND_F32, D, 1),
             ("sgate", None): (uq.KIND_Q8_0, D, FF), ("sup", None): (uq.KIND_Q8_0, D, FF),
             ("sdown", None): (uq.KIND_Q8_0, FF, D)}
    for e in range(E):
        specs[("gate", e)] = (uq.KIND_IQ3_XXS, D, FF)
        specs[("up", e)] = (uq.KIND_IQ3_XXS, D, FF)
        specs[("down", e)] = (uq.KIND_IQ4_NL, FF, D)
    raw, weights = {}, {}
    for i, (key, (kind, n, m)) in enumerate(sorted(specs.items(), key=lambda kv: str(kv[0]))):
        r = uq.synth_quant(kind, 0xF0E0 + i, m, n)
        raw[key] = (kind, n, m, r)
        weights[key] = uq.Weight(kind, n, m, r)
    yield raw, weights
    for w in weights.values():
        w.free()


def test_frontier_ffn_matches_oracle_composition(bank):
    raw, weights = bank

    def g_linear(key, x):
        return uq.linear(weights[key], x)

    def g_batch(reqs):
        return uq.linear_batch([(weights[k], x) for k, x in reqs])

    def o_linear(key, x):
        kind, n, m, r = raw[key]
        return O.linear(kind, r, n, m, x)

    def o_batch(reqs):
        return [o_linear(k, x) for k, x in reqs]

    for seed in (1, 2, 3):
        x = uq.synth_normal(0xF1 + seed, D, 0.0, 1.0)
        got, gids = ffn(g_linear, g_batch, weights, x)
        ref, rids = ffn(o_linear, o_batch, weights, x)
        assert gids == rids
        assert np.isfinite(got).all()
        assert np.abs(got - ref).max() <= 1e-3 * np.abs(ref).max(), np.abs(got - ref).max()


def test_frontier_batches_equal_single_linears(bank):
    _, weights = bank
    x = uq.synth_normal(0xF9, D, 0.0, 1.0)
    reqs = [(weights[("gate", e)], x) for e in range(0, 20, 2)] + [(weights[("up", e)], x) for e in range(5)]
    for (w, xx), y in zip(reqs, uq.linear_batch(reqs)):
        assert np.array_equal(y.view(np.uint32), uq.linear(w, xx).view(np.uint32))
