"""Writes tests/golden/qwen25_refo.npz: logits of the reference-order decoder
(oracle/uq_oracle.c uqo_refo_*, the f32 operation orders of the reference's
decode-graph kernels) on the 28-layer Qwen2.5-1.5B-architecture synthetic
model of qwen25_decode.json (seed 0x5EED0002), teacher-forced: the 512-token
prompt token by token, then all 128 decode steps of that fixture, fed
[first_id] + ids[:127] (the build's own greedy ids, so the forced run is the
free-running greedy run of the exact contract).

Saved for the 129 positions 511..639 (the prompt's last token, then the forced
steps), once with an f32 KV cache (the reference's) and once with the cache
rounded to fp16 (the library's format):
  idx        the compared vocabulary ids per position: the 64 largest logits
             of the f32-cache run, then 192 fixed seeded ids
  ref_f32, ref_f16   those logits
  absmax_*, argmax_*, margin_*  max |logit|, argmax and top-2 margin per run
  argmax_exact, margin_exact    the same of the exact-double oracle
  exact_dev  max |exact-oracle logit - reference-order logit| / max |logit|
             over the compared ids (fp16 cache), for the record

Usage: python tests/golden/make_refo_golden.py
"""
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


def main():
    g = json.load(open(os.path.join(HERE, "qwen25_decode.json")))
    cfg, seed, n = g["config"], g["seed"], g["prompt_len"]
    t = uq.synth_qwen2(cfg, seed)
    arrays = {k: v[3] for k, v in t.items()}
    prompt = uq.synth_tokens(seed, n, cfg["vocab"])
    forced = [g["first_id"]] + g["ids"][:127]
    rng = np.random.default_rng(0x5EED0077)
    sample = np.sort(rng.choice(cfg["vocab"], 192, replace=False))
    runs = {}
    for name, kv16 in (("f32", False), ("f16", True)):
        t0 = time.time()
        m = O.RefoModel(cfg, arrays, kv_fp16=kv16)
        logits = []
        for pos, tok in enumerate(list(prompt) + forced):
            want = pos >= n - 1
            rc, _, lg = m.decode(int(tok), pos, want_logits=want)
            assert rc == 0, (name, pos, rc)
            if want:
                logits.append(lg)
        runs[name] = np.stack(logits)
        print(name, "%.1f s" % (time.time() - t0), flush=True)
        del m
    idx = np.stack([np.concatenate([np.argsort(r)[-64:], sample]) for r in runs["f32"]])
    # the exact oracle under the same forcing: prefill, then the forced steps
    ex = O.Model(cfg, arrays)
    rc, _, lg = ex.prefill(prompt, want_logits=True)
    exact = [lg]
    for i, tok in enumerate(forced):
        rc, _, lg = ex.decode(int(tok), n + i, want_logits=True)
        exact.append(lg)
    exact = np.stack(exact)
    out = {"idx": idx.astype(np.int32)}
    for name in ("f32", "f16"):
        r = runs[name]
        out["ref_" + name] = np.take_along_axis(r, idx, 1).astype(np.float32)
        out["absmax_" + name] = np.abs(r).max(1).astype(np.float32)
        out["argmax_" + name] = r.argmax(1).astype(np.int32)
        s = np.sort(r, 1)
        out["margin_" + name] = (s[:, -1] - s[:, -2]).astype(np.float32)
    dev = np.abs(np.take_along_axis(exact, idx, 1) - out["ref_f16"]).max(1) / out["absmax_f16"]
    out["exact_dev"] = dev.astype(np.float32)
    out["argmax_exact"] = exact.argmax(1).astype(np.int32)
    s = np.sort(exact, 1)
    out["margin_exact"] = (s[:, -1] - s[:, -2]).astype(np.float32)
    out["forced"] = np.array(forced, np.int32)
    np.savez_compressed(os.path.join(HERE, "qwen25_refo.npz"), **out)
    print("exact vs reference-order (fp16 cache) max dev per position:", np.round(dev, 4))
    for k in ("f32", "f16"):
        agree = out["argmax_exact"] == out["argmax_" + k]
        rel = out["margin_" + k] / out["absmax_" + k]
        print("ids equal to the %s-cache reference order: %d of %d; smallest top-2 margin/max|logit| %.2e, "
              "largest where they differ %.2e" % (k, agree.sum(), agree.size, rel.min(),
                                                  rel[~agree].max() if (~agree).any() else 0.0))
    agree = out["argmax_f32"] == out["argmax_f16"]
    print("f32-cache vs fp16-cache reference order: ids equal at %d of %d" % (agree.sum(), agree.size))


if __name__ == "__main__":
    main()
