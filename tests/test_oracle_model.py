"""Pins the oracle's Qwen2 decoder wiring (residuals, biases, RoPE pairs, GQA
head mapping, SwiGLU, output head) against an independent numpy float64
restatement of driver/src/llm.rs:339-388 that only shares the int8 activation
quantization rule, and checks prefill/decode consistency inside the oracle."""
import numpy as np
import pytest

import oracle as O
import uq
import ggml_layouts as G

TINY = dict(layers=2, dim=256, hidden=512, heads=4, kv_heads=2, head_dim=64, vocab=500, max_seq=32,
            eps=1e-6, theta=1e6)


def np_quant(x):
    b = x.astype(np.float32).reshape(-1, 32)
    a = np.abs(b).max(1)
    inv = np.where(a > 0, np.float32(127) / np.where(a > 0, a, 1), 0).astype(np.float32)
    q = np.clip(np.rint((b * inv[:, None]).astype(np.float32)), -127, 127)
    return (q * (a / np.float32(127))[:, None]).reshape(-1).astype(np.float64)


class NumpyQwen2:
    def __init__(self, cfg, t):
        self.c = cfg
        self.W = {}
        for name, (kind, n, rows, arr) in t.items():
            self.W[name] = G.q8_0_dequant(arr, rows, n).astype(np.float64) if kind == uq.KIND_Q8_0 \
                else arr.astype(np.float64)
        L, S, kvd = cfg["layers"], cfg["max_seq"], cfg["kv_heads"] * cfg["head_dim"]
        self.K = np.zeros((L, S, kvd))
        self.V = np.zeros((L, S, kvd))

    def rope(self, v, heads, pos):
        hd = self.c["head_dim"]
        i = np.arange(hd // 2)
        ang = pos * self.c["theta"] ** (-(2 * i) / hd)
        v = v.reshape(heads, hd).copy()
        a, b = v[:, :hd // 2].copy(), v[:, hd // 2:].copy()
        v[:, :hd // 2] = a * np.cos(ang) - b * np.sin(ang)
        v[:, hd // 2:] = a * np.sin(ang) + b * np.cos(ang)
        return v.reshape(-1)

    def norm(self, x, w):
        return x / np.sqrt((x * x).mean() + self.c["eps"]) * w

    def step(self, token, pos):
        c, W = self.c, self.W
        hd, H, KV = c["head_dim"], c["heads"], c["kv_heads"]
        x = W["token_embd.weight"][token].copy()
        for l in range(c["layers"]):
            p = lambda s: W["blk.%d.%s" % (l, s)]
            xn = np_quant(self.norm(x, p("attn_norm.weight")))
            q = self.rope(p("attn_q.weight") @ xn + p("attn_q.bias"), H, pos)
            k = self.rope(p("attn_k.weight") @ xn + p("attn_k.bias"), KV, pos)
            v = p("attn_v.weight") @ xn + p("attn_v.bias")
            self.K[l, pos] = k.astype(np.float16)
            self.V[l, pos] = v.astype(np.float16)
            att = np.zeros(c["dim"])
            for h in range(H):
                kh = h // (H // KV)
                Ks = self.K[l, :pos + 1, kh * hd:(kh + 1) * hd]
                s = Ks @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
                pr = np.exp(s - s.max())
                pr /= pr.sum()
                att[h * hd:(h + 1) * hd] = pr @ self.V[l, :pos + 1, kh * hd:(kh + 1) * hd]
            x = x + p("attn_output.weight") @ np_quant(att)
            xn = np_quant(self.norm(x, p("ffn_norm.weight")))
            g, u = p("ffn_gate.weight") @ xn, p("ffn_up.weight") @ xn
            x = x + p("ffn_down.weight") @ np_quant(g / (1 + np.exp(-g)) * u)
        xn = np_quant(self.norm(x, W["output_norm.weight"]))
        return W["output.weight"] @ xn


def test_oracle_decoder_matches_numpy_restatement():
    t = uq.synth_qwen2(TINY, 11)
    o = O.Model(TINY, {k: v[3] for k, v in t.items()})
    ref = NumpyQwen2(TINY, t)
    toks = uq.synth_tokens(11, 5, TINY["vocab"])
    for pos, tok in enumerate(toks):
        rc, nxt, lg = o.decode(int(tok), pos, want_logits=True)
        assert rc == 0
        r = ref.step(int(tok), pos)
        scale = np.abs(r).max()
        assert np.abs(lg - r).max() < 2e-3 * scale, (pos, np.abs(lg - r).max(), scale)
        assert nxt == int(np.argmax(lg))


def test_oracle_prefill_matches_decode_chain():
    t = uq.synth_qwen2(TINY, 12)
    arrays = {k: v[3] for k, v in t.items()}
    toks = uq.synth_tokens(12, 20, TINY["vocab"])
    a = O.Model(TINY, arrays)
    rc, nxt_p, lg_p = a.prefill(toks, want_logits=True)
    assert rc == 0
    b = O.Model(TINY, arrays)
    for pos, tok in enumerate(toks):
        rc, nxt_d, lg_d = b.decode(int(tok), pos, want_logits=True)
        assert rc == 0
    # GEMM-order (sequential fmaf) and decode-order (exact sum) linears differ
    # only by f32 rounding; quantization may amplify a rare tie flip
    scale = np.abs(lg_d).max()
    assert np.abs(lg_p - lg_d).max() < 2e-3 * scale
    for layer in range(TINY["layers"]):
        kp = a.keys(layer, 20).view(np.float16).astype(np.float32)
        kd = b.keys(layer, 20).view(np.float16).astype(np.float32)
        assert np.abs(kp - kd).max() <= 2e-3 * np.abs(kd).max()
    # a second prefill over the same prompt is deterministic
    c = O.Model(TINY, arrays)
    assert c.prefill(toks, want_logits=True)[1] == nxt_p


@pytest.mark.parametrize("gated", [True, False])
def test_oracle_moe_matches_numpy_restatement(gated):
    """frontier_forward.rs:164-199 restated in numpy float64 around the shared
    int8 activation rule: softmax, stable top-k, p/sum weights, SwiGLU experts,
    rank-ordered combine, sigmoid-gated shared expert (weight 1 for a layer
    without ffn_gate_inp_shexp)."""
    cfg = dict(dim=256, ff=256, experts=8, top_k=2, expert_kind=uq.KIND_Q8_0, shared_kind=uq.KIND_Q8_0)
    ex, sh, gi = uq.synth_moe(cfg, 3)
    if not gated:
        gi = None
    om = O.MoeLayer(cfg["dim"], cfg["ff"], cfg["experts"], cfg["top_k"], cfg["expert_kind"],
                    [e[0] for e in ex], [e[1] for e in ex], [e[2] for e in ex], cfg["shared_kind"],
                    sh[0], sh[1], sh[2], gi)
    D, F = cfg["dim"], cfg["ff"]
    deq = lambda raw, rows, n: G.q8_0_dequant(raw, rows, n).astype(np.float64)
    for step in range(4):
        x = uq.synth_normal(50 + step, D)
        lg = uq.synth_normal(60 + step, cfg["experts"])
        rc, out, ids, w = om.ffn(x, lg)
        assert rc == 0
        p = np.exp(lg.astype(np.float64) - lg.max())
        p /= p.sum()
        order = sorted(range(cfg["experts"]), key=lambda e: (-np.float32(p[e]), e))[:cfg["top_k"]]
        assert list(ids) == order
        wts = p[order] / p[order].sum()
        xq = np_quant(x)
        ref = np.zeros(D)

        def expert(g, u, d):
            gv, uv = deq(g, F, D) @ xq, deq(u, F, D) @ xq
            mid = gv / (1 + np.exp(-gv)) * uv
            return deq(d, D, F) @ np_quant(mid)
        for r, e in enumerate(order):
            ref += wts[r] * expert(*ex[e])
        sw = 1.0 if gi is None else 1 / (1 + np.exp(-(gi.astype(np.float64) @ x.astype(np.float64))))
        ref += sw * expert(*sh)
        assert np.abs(out - ref).max() < 2e-3 * np.abs(ref).max()


def test_oracle_reproduces_committed_fixtures():
    """tests/golden/small.npz was written by tests/golden/make_golden.py; the
    oracle must reproduce every output bit for bit."""
    import os
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "small.npz"))
    q, s = O.quant_act(f["quant_x"])
    assert np.array_equal(q, f["quant_q"]) and np.array_equal(s, f["quant_s"])
    for kind, name, n, m in ((O.Q8_0, "q8", 256, 64), (O.Q4_K, "q4k", 512, 48), (O.Q3_K, "q3k", 512, 40)):
        y = O.matvec(kind, f[name + "_w"], n, m, f[name + "_x"])
        assert np.array_equal(y, f[name + "_y"])
        qx, _ = O.quant_act(f[name + "_x"])
        assert np.array_equal(O.block_dots(kind, f[name + "_w"], n, m, qx), f[name + "_dots"])
    y = O.prefill_gemm(f["q8_w"], 256, 64, f["gemm_xs"], f["gemm_qx"], 70)
    assert np.array_equal(y, f["gemm_y"])
    out = O.attention(f["attn_q"], f["attn_k"], f["attn_v"], 39, 12, 2, 128)
    assert np.array_equal(out, f["attn_out"])
