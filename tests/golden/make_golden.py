"""Writes the committed golden fixtures of this path from the CPU oracle.

The reference repository holds no vectors for its hot path (its checks are
live on-device gates), so the fixtures here are produced by the oracle
(oracle/uq_oracle.c) on seeded synthetic inputs from the package generator:

  small.npz   small Q8_0 / Q4_K / Q3_K matvecs, activation quant, prefill GEMM,
              attention and MoE cases with their inputs and outputs
  qwen25_decode.json  Qwen2.5-1.5B-architecture greedy run (random-init Q8_0
              weights, seed 0x5EED0002): 512-token prompt through the prefill,
              then 128 decode steps; token ids and per-step top-2 margins

Usage: python tests/golden/make_golden.py [--skip-model]
"""
import argparse
import hashlib
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "uefi-gpu_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import numpy as np  # noqa: E402

import oracle as O  # noqa: E402
import uq  # noqa: E402


def small_fixtures():
    out = {}
    # activation quant (ties, zeros, amax)
    x = uq.synth_normal(1, 512)
    x[:32] = 0
    x[32] = 127.0
    x[33:41] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5]
    q, s = O.quant_act(x)
    out.update(quant_x=x, quant_q=q, quant_s=s)
    for kind, name, n, m in ((O.Q8_0, "q8", 256, 64), (O.Q4_K, "q4k", 512, 48), (O.Q3_K, "q3k", 512, 40)):
        w = uq.synth_quant(kind, 0x5EED0000 + kind, m, n)
        xv = uq.synth_normal(0x5EED0100 + kind, n)
        out[name + "_w"] = w
        out[name + "_x"] = xv
        out[name + "_y"] = O.matvec(kind, w, n, m, xv)
        qx, _ = O.quant_act(xv)
        out[name + "_dots"] = O.block_dots(kind, w, n, m, qx)
    # prefill GEMM: 70 tokens x 64 rows x K 256
    w = out["q8_w"]
    X = np.stack([uq.synth_normal(0x5EED0200 + t, 256) for t in range(70)])
    qs = [O.quant_act(r) for r in X]
    qx = np.stack([a for a, _ in qs])
    xs = np.stack([b for _, b in qs])
    out.update(gemm_qx=qx, gemm_xs=xs, gemm_y=O.prefill_gemm(w, 256, 64, xs, qx, 70))
    # attention over an fp16 cache
    qv = uq.synth_normal(0x5EED0300, 12 * 128, 0.0, 3.0)
    K = uq.synth_normal(0x5EED0301, 40 * 256, 0.0, 3.0).astype(np.float16).view(np.uint16)
    V = uq.synth_normal(0x5EED0302, 40 * 256, 0.0, 3.0).astype(np.float16).view(np.uint16)
    out.update(attn_q=qv, attn_k=K, attn_v=V, attn_out=O.attention(qv, K, V, 39, 12, 2, 128))
    return out


def qwen25_run(prompt_len=512, steps=128, threads=8):
    O.set_threads(threads)
    cfg = dict(uq.QWEN25_15B, max_seq=1024)
    seed = 0x5EED0002
    t = uq.synth_qwen2(cfg, seed)
    digest = hashlib.sha256()
    for name in sorted(t):
        digest.update(name.encode())
        digest.update(hashlib.sha256(t[name][3].tobytes()).digest())
    model = O.Model(cfg, {k: v[3] for k, v in t.items()})
    prompt = uq.synth_tokens(seed, prompt_len, cfg["vocab"])
    t0 = time.time()
    rc, first, lg = model.prefill(prompt, want_logits=True)
    assert rc == 0, rc
    t_prefill = time.time() - t0
    ids, margins = [int(first)], []
    srt = np.sort(lg)
    margins.append(float(srt[-1] - srt[-2]))
    tok = int(first)
    for i in range(steps):
        rc, tok, lg = model.decode(tok, prompt_len + i, want_logits=True)
        assert rc == 0, rc
        ids.append(int(tok))
        srt = np.sort(lg)
        margins.append(float(srt[-1] - srt[-2]))
    return {"config": cfg, "seed": seed, "prompt_len": prompt_len, "steps": steps,
            "weights_sha256": digest.hexdigest(),
            "prompt_sha256": hashlib.sha256(prompt.tobytes()).hexdigest(),
            "ids": ids[1:], "first_id": ids[0], "top2_margins": margins,
            "note": "ids[i] is the greedy id produced at position prompt_len + i; first_id after the prompt",
            "oracle_prefill_s": round(t_prefill, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--skip-model", action="store_true")
    args = ap.parse_args()
    np.savez_compressed(os.path.join(HERE, "small.npz"), **small_fixtures())
    print("wrote small.npz", flush=True)
    if not args.skip_model:
        res = qwen25_run()
        with open(os.path.join(HERE, "qwen25_decode.json"), "w") as f:
            json.dump(res, f, indent=1)
        print("wrote qwen25_decode.json", res["first_id"], res["ids"][:8], flush=True)


if __name__ == "__main__":
    main()
