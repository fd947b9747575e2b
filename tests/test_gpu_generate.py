"""uq_generate (generate_one, driver/src/llm.rs:402-428) on the GPU: the same
ids as the oracle's prefill followed by its greedy decode chain, the same ids
as the library's own prefill followed by device-fed decode steps, the stop-id
and limit rules of the reference loop, and the eval runner over the
reference's prompt files with a synthetic vocabulary."""
import os

import numpy as np
import pytest

import gguf_writer as W
import oracle as O
import uq
import evalrun

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
PROMPTS = os.path.join(HERE, "golden", "prompts")
CFG = dict(uq.QWEN25_15B, layers=2, max_seq=256)


@pytest.fixture(scope="module")
def tensors():
    return uq.synth_qwen2(CFG, 0x6E0)


@pytest.fixture(scope="module")
def model(gpu, tensors):
    m = uq.Qwen2Model(CFG, tensors)
    yield m
    m.free()


def oracle_chain(tensors, prompt, n):
    """generate_one's loop (llm.rs:402-428) on the oracle decoder: prefill the
    prompt, then feed each greedy id back as the next token."""
    o = O.Model(CFG, {k: v[3] for k, v in tensors.items()})
    rc, tok, _ = o.prefill(prompt)
    assert rc == 0
    ids = [tok]
    for pos in range(len(prompt), len(prompt) + n - 1):
        rc, tok, _ = o.decode(tok, pos)
        assert rc == 0
        ids.append(tok)
    return np.array(ids, np.uint32)


def reference_chain(model, prompt, n):
    """prefill, then n-1 decode steps fed back on the device."""
    first = model.prefill(prompt)
    if n == 1:
        return np.array([first], np.uint32)
    rest, _ = model.decode_run(first, len(prompt), n - 1)
    return np.concatenate([[first], rest]).astype(np.uint32)


def test_generate_matches_oracle_and_prefill_decode(model, tensors):
    prompt = evalrun.read_tokens(os.path.join(PROMPTS, "prompt_sentence.tokens"))
    ids, ended, pms, dms = model.generate(prompt, 40, stop=())
    assert len(ids) == 40 and not ended and pms > 0 and dms > 0
    assert np.array_equal(ids, oracle_chain(tensors, prompt, 40))
    assert np.array_equal(ids, reference_chain(model, prompt, 40))


def test_stop_ids_and_limit(model):
    prompt = evalrun.read_tokens(os.path.join(PROMPTS, "prompt_riddle.tokens"))
    ref = reference_chain(model, prompt, 12)
    # a stop id that is the first id: nothing emitted, ended
    ids, ended, _, _ = model.generate(prompt, 12, stop=(int(ref[0]),))
    assert len(ids) == 0 and ended
    # stop at the first occurrence of ref[5]: the ids before it
    k = int(np.nonzero(ref == ref[5])[0][0])
    ids, ended, _, _ = model.generate(prompt, 12, stop=(int(ref[5]),))
    assert ended and np.array_equal(ids, ref[:k])
    # the limit: exactly max_new ids, not ended
    ids, ended, _, _ = model.generate(prompt, 12, stop=())
    assert np.array_equal(ids, ref[:12]) and not ended
    with pytest.raises(uq.UqError) as e:
        model.generate(prompt, CFG["max_seq"] - len(prompt), stop=())
    assert e.value.status == uq.Error.CONTEXT


def test_eval_runner_lines(model):
    # a vocabulary whose token i is "w<i>" + GPT-2 space: text is the ids joined
    vocab_tokens = ["w%dĠ" % i for i in range(CFG["vocab"])]
    data, _ = W.write([("tokenizer.ggml.tokens", W.ARRAY, (W.STRING, vocab_tokens))], [])
    vocab = uq.Gguf.parse(np.frombuffer(data, np.uint8), len(data))
    prompt = evalrun.read_tokens(os.path.join(PROMPTS, "prompt_sentence.tokens"))
    lines = []
    r = evalrun.run_prompt(model, prompt, "sentence", "prompt text", vocab, max_new=16, emit=lines.append)
    ids = reference_chain(model, prompt, 16)
    # an end id of the reference may appear in the synthetic run: the output stops before it
    end = [i for i, t in enumerate(ids) if int(t) in evalrun.END_IDS]
    want = ids[:end[0]] if end else ids
    assert np.array_equal(r["ids"], want)
    assert r["text"] == "".join("w%d " % int(t) for t in want)
    assert lines[0] == "LLM PROMPT sentence: prompt text"
    assert lines[1].startswith("BENCH prompt=sentence phase=prefill tokens=28 ")
    assert lines[2].startswith("BENCH prompt=sentence phase=decode tokens=%d " % len(want))
    assert lines[3].startswith("LLM OUTPUT sentence tokens=%d eos=%s: " % (len(want), str(bool(end)).lower()))
