"""Pins the oracle's Qwen2 decoder wiring (residuals, biases, RoPE pairs, GQA
head mapping, SwiGLU, output head) against an independent numpy float64
restatement of driver/src/llm.rs:339-388 that only shares the int8 activation
quantization rule, and checks prefill/decode consistency inside the oracle."""
import numpy as np

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
