"""Prompt runs of the reference's `generate` (driver/src/llm.rs:396-447) over the
uq C ABI: packed prompt token files, prefill, greedy decode to an end id or
the token limit, detokenized output and per-phase timing lines.

    python uefi-gpu_amd/evalrun.py --gguf model.gguf --prompts DIR [--max-seq 1024]
    python uefi-gpu_amd/evalrun.py --synthetic --prompts DIR

`--gguf` loads a Qwen2 GGUF (weights and tokenizer.ggml.tokens); `--synthetic`
builds the seeded random-init Qwen2.5-1.5B-shape model and prints token ids
instead of text. DIR holds prompt_<label>.tokens (u32 count, then count u32
ids, little-endian) and prompt_<label>.txt, the files of driver/models/.
"""
import argparse
import os
import struct
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import uq  # noqa: E402

END_IDS = (151645, 151643)        # <|im_end|>, <|endoftext|> (llm.rs:424,429)
LABELS = ("sentence", "riddle", "scale")


def read_tokens(path):
    """The packed prompt of llm.rs:403-405: u32 count, then count u32 ids."""
    raw = open(path, "rb").read()
    if len(raw) < 4:
        raise ValueError("%s: no count" % path)
    (count,) = struct.unpack_from("<I", raw, 0)
    if len(raw) != 4 + 4 * count:
        raise ValueError("%s: count %d does not match %d id bytes" % (path, count, len(raw) - 4))
    return np.frombuffer(raw, np.uint32, count, 4).copy()


def max_new_for(label):
    """Token limit of llm.rs:406: 512 for the long prompt, 160 otherwise."""
    return 512 if label == "scale" else 160


def run_prompt(model, tokens, label, prompt_text, vocab=None, max_new=None, emit=print):
    """One generate_one: returns a dict of the run and emits the reference's lines."""
    if max_new is None:
        max_new = max_new_for(label)
    ids, ended, prefill_ms, decode_ms = model.generate(tokens, max_new, END_IDS)
    n = len(ids)
    text = "".join(vocab.text(int(t)) for t in ids) if vocab is not None else " ".join(str(int(t)) for t in ids)
    emit("LLM PROMPT %s: %s" % (label, prompt_text))
    for phase, count, ms in (("prefill", len(tokens), prefill_ms), ("decode", n, decode_ms)):
        ns = int(ms * 1e6)
        per = ms / count if count else 0.0
        tps = count * 1e3 / ms if ms > 0 else 0.0
        emit("BENCH prompt=%s phase=%s tokens=%d elapsed_ns=%d ms_per_token=%.6f tokens_per_sec=%.6f"
             % (label, phase, count, ns, per, tps))
    emit("LLM OUTPUT %s tokens=%d eos=%s: %s" % (label, n, str(ended).lower(), text))
    emit("GENERATION_LIMIT prompt=%s limit=%d reached=%s final_position=%d"
         % (label, max_new, str(not ended and n == max_new).lower(), len(tokens) + n))
    return {"label": label, "ids": ids, "ended": ended, "text": text, "prefill_ms": prefill_ms,
            "decode_ms": decode_ms}


def main(argv=None):
    ap = argparse.ArgumentParser()
    src = ap.add_mutually_exclusive_group(required=True)
    src.add_argument("--gguf", help="Qwen2 GGUF file (weights and tokenizer)")
    src.add_argument("--synthetic", action="store_true", help="seeded random-init Qwen2.5-1.5B-shape model")
    ap.add_argument("--prompts", required=True, help="directory of prompt_<label>.tokens / .txt")
    ap.add_argument("--max-seq", type=int, default=1024)
    ap.add_argument("--labels", default=",".join(LABELS))
    args = ap.parse_args(argv)
    uq.init(0)
    vocab = None
    if args.gguf:
        vocab = uq.Gguf.open(args.gguf)
        model = uq.Qwen2Model.from_gguf(args.gguf, max_seq=args.max_seq)
    else:
        cfg = dict(uq.QWEN25_15B, max_seq=args.max_seq)
        model = uq.Qwen2Model(cfg, uq.synth_qwen2(cfg, 0x5EED0003))
    for label in args.labels.split(","):
        tokens = read_tokens(os.path.join(args.prompts, "prompt_%s.tokens" % label))
        with open(os.path.join(args.prompts, "prompt_%s.txt" % label), encoding="utf-8") as f:
            prompt_text = f.read()
        run_prompt(model, tokens, label, prompt_text, vocab)
    model.free()
    return 0


if __name__ == "__main__":
    sys.exit(main())
